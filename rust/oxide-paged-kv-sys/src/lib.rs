//! Raw FFI bindings of `liboxide_paged_kv` -- the gfx950 (MI355X) kernels of vllm-oxide's
//! paged-KV path -- declared in `include/oxide_paged_kv.h` and `include/oxide_workload.h`.
//!
//! This replaces the `extern "C"` block of crates/vllm-oxide/src/attention/kernels.rs:10-38:
//! `reshape_and_cache` and `copy_blocks` keep the reference's symbols and parameter lists
//! (`c_long` as there), the stream is a `hipStream_t` where the reference passes a
//! `CUstream`, and the remaining entries are the new calls of the path (decode and prefill
//! attention over the paged cache, the fused prologue, device metadata, the gather).
//!
//! With the `rocm` feature, build.rs compiles the HIP sources with hipcc for gfx950 into a
//! static `liboxide_paged_kv.a` and links it with amdhip64; without it nothing is linked,
//! as the reference's kernels are absent without its `cuda` feature.
//!
//! Every call is asynchronous on the given stream and returns nothing (as the reference's
//! do); argument and launch errors are read back with `oxide_last_error()` on the calling
//! thread.  All pointers are device pointers unless a comment says host.
#![no_std]

use core::ffi::{c_char, c_int, c_long, c_void};

/// `hipStream_t` (null = the default stream).
pub type HipStream = *mut c_void;

/// dtype codes (crates/vllm-oxide/src/attention/kernels.rs:97-104).
pub const OXIDE_DTYPE_F16: c_int = 0;
pub const OXIDE_DTYPE_BF16: c_int = 1;
pub const OXIDE_DTYPE_F32: c_int = 2;

/// Error codes of `oxide_last_error`; a failed launch reads OXIDE_ERR_HIP + its hipError_t.
pub const OXIDE_OK: c_int = 0;
pub const OXIDE_ERR_INVALID_ARGUMENT: c_int = 1;
pub const OXIDE_ERR_UNSUPPORTED_DTYPE: c_int = 2;
pub const OXIDE_ERR_UNSUPPORTED_SHAPE: c_int = 3;
pub const OXIDE_ERR_WORKSPACE_TOO_SMALL: c_int = 4;
pub const OXIDE_ERR_SCRATCH_TOO_SMALL: c_int = 5;
pub const OXIDE_ERR_HIP: c_int = 1000;

extern "C" {
    /// KV append; same symbol and parameters as crates/vllm-oxide/kernels/reshape_and_cache.cu:30-41
    /// (bound at crates/vllm-oxide/src/attention/kernels.rs:15-26), `stream` a hipStream_t.
    pub fn reshape_and_cache(
        key: *const c_void,
        value: *const c_void,
        key_cache: *mut c_void,
        value_cache: *mut c_void,
        slot_mapping: *const c_long,
        num_tokens: c_long,
        num_kv_heads: c_long,
        head_dim: c_long,
        dtype: c_int,
        stream: HipStream,
    );

    /// Copy-on-write block copy; same symbol and parameters as crates/vllm-oxide/kernels/copy_blocks.cu:30-38
    /// (kernels.rs:28-36).  `block_stride` in elements; dst blocks disjoint from src blocks.
    pub fn copy_blocks(
        key_cache: *mut c_void,
        value_cache: *mut c_void,
        block_mapping: *const c_long,
        num_pairs: c_long,
        block_stride: c_long,
        dtype: c_int,
        stream: HipStream,
    );

    /// Prefix-hit gather of whole blocks into contiguous K/V (no reference counterpart).
    pub fn gather_blocks(
        key_dst: *mut c_void,
        value_dst: *mut c_void,
        key_cache: *const c_void,
        value_cache: *const c_void,
        block_ids: *const i32,
        num_blocks: i64,
        block_stride: i64,
        dtype: c_int,
        stream: HipStream,
    );

    /// The decode call of flash_attn_varlen_paged_windowed (crates/vllm-oxide/src/attention/flash_attn.rs:52-67):
    /// GQA, left window (-1 = none), split-KV with a caller-owned workspace.
    pub fn paged_decode_attention(
        out: *mut c_void,
        q: *const c_void,
        k_cache: *const c_void,
        v_cache: *const c_void,
        cu_seqlens_k: *const u32,
        block_table: *const i32,
        max_blocks_per_seq: i64,
        num_blocks: i64,
        batch: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        page_block_size: i64,
        max_seqlen_k: i64,
        window_left: i32,
        softmax_scale: f32,
        workspace: *mut c_void,
        workspace_bytes: usize,
        dtype: c_int,
        stream: HipStream,
    );

    /// reshape_and_cache + paged_decode_attention in one launch (the append-then-attend order of
    /// crates/vllm-oxide/src/models/qwen3.rs:199-208).
    pub fn paged_decode_attention_append(
        out: *mut c_void,
        q: *const c_void,
        key: *const c_void,
        value: *const c_void,
        slot_mapping: *const i64,
        k_cache: *mut c_void,
        v_cache: *mut c_void,
        cu_seqlens_k: *const u32,
        block_table: *const i32,
        max_blocks_per_seq: i64,
        num_blocks: i64,
        batch: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        page_block_size: i64,
        max_seqlen_k: i64,
        window_left: i32,
        softmax_scale: f32,
        workspace: *mut c_void,
        workspace_bytes: usize,
        dtype: c_int,
        stream: HipStream,
    );

    /// Workspace bytes for paged_decode_attention / _append / _path with these arguments.
    pub fn paged_decode_attention_workspace_size(
        batch: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        max_seqlen_k: i64,
    ) -> usize;

    /// First pass chosen by shape: split size (> 0), 0 persistent, -1 stream.
    pub fn paged_decode_attention_split_tokens(
        batch: i64,
        num_kv_heads: i64,
        max_seqlen_k: i64,
    ) -> i64;

    /// Tuning / tests: the decode calls with the first pass chosen for this call only
    /// (0 by shape, 1 split, 2 persistent, 3 stream); key/value/slot_mapping all null = no append.
    pub fn paged_decode_attention_path(
        path: c_int,
        out: *mut c_void,
        q: *const c_void,
        key: *const c_void,
        value: *const c_void,
        slot_mapping: *const i64,
        k_cache: *mut c_void,
        v_cache: *mut c_void,
        cu_seqlens_k: *const u32,
        block_table: *const i32,
        max_blocks_per_seq: i64,
        num_blocks: i64,
        batch: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        page_block_size: i64,
        max_seqlen_k: i64,
        window_left: i32,
        softmax_scale: f32,
        workspace: *mut c_void,
        workspace_bytes: usize,
        dtype: c_int,
        stream: HipStream,
    );

    /// paged_decode_attention_split_tokens for a forced first pass.
    pub fn paged_decode_attention_path_split_tokens(
        path: c_int,
        batch: i64,
        num_kv_heads: i64,
        max_seqlen_k: i64,
    ) -> i64;

    /// Cascaded decode for batches whose block-table rows share leading entries (a cached
    /// prompt prefix): the shared keys attended once for all sequences, the rest per sequence;
    /// key/value/slot_mapping all null = no append.  No reference counterpart.
    pub fn paged_decode_attention_shared_prefix(
        out: *mut c_void,
        q: *const c_void,
        key: *const c_void,
        value: *const c_void,
        slot_mapping: *const i64,
        k_cache: *mut c_void,
        v_cache: *mut c_void,
        cu_seqlens_k: *const u32,
        block_table: *const i32,
        max_blocks_per_seq: i64,
        num_blocks: i64,
        batch: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        page_block_size: i64,
        max_seqlen_k: i64,
        window_left: i32,
        softmax_scale: f32,
        shared_blocks_hint: i64,
        workspace: *mut c_void,
        workspace_bytes: usize,
        dtype: c_int,
        stream: HipStream,
    );

    /// paged_decode_attention_shared_prefix with its form given: 0 by shape, 1 cascade one pass
    /// after the other, 2 cascade overlapped, 3 plain entries.
    pub fn paged_decode_attention_shared_prefix_mode(
        mode: c_int,
        out: *mut c_void,
        q: *const c_void,
        key: *const c_void,
        value: *const c_void,
        slot_mapping: *const i64,
        k_cache: *mut c_void,
        v_cache: *mut c_void,
        cu_seqlens_k: *const u32,
        block_table: *const i32,
        max_blocks_per_seq: i64,
        num_blocks: i64,
        batch: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        page_block_size: i64,
        max_seqlen_k: i64,
        window_left: i32,
        softmax_scale: f32,
        shared_blocks_hint: i64,
        workspace: *mut c_void,
        workspace_bytes: usize,
        dtype: c_int,
        stream: HipStream,
    );

    /// The form paged_decode_attention_shared_prefix takes: 1, 2 or 3 as above.
    pub fn paged_decode_attention_shared_prefix_plan(
        batch: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        page_block_size: i64,
        max_seqlen_k: i64,
        shared_blocks_hint: i64,
    ) -> c_int;

    pub fn paged_decode_attention_shared_prefix_workspace_size(
        batch: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        page_block_size: i64,
        max_seqlen_k: i64,
        shared_blocks_hint: i64,
    ) -> usize;

    /// First pass run by paged_decode_attention_path(path, ...): split size (> 0), 0 persistent,
    /// -1 stream, -2 row pass.
    pub fn paged_decode_attention_pass1(
        path: c_int,
        batch: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        page_block_size: i64,
        max_seqlen_k: i64,
    ) -> i64;

    /// Prefill (seqlen_q >= 1) call of flash_attn_varlen_paged_windowed over the paged cache, causal,
    /// masks aligned bottom-right; cached prefix keys are read in place.
    pub fn paged_prefill_attention(
        out: *mut c_void,
        q: *const c_void,
        k_cache: *const c_void,
        v_cache: *const c_void,
        cu_seqlens_q: *const u32,
        cu_seqlens_k: *const u32,
        block_table: *const i32,
        max_blocks_per_seq: i64,
        num_blocks: i64,
        batch: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        page_block_size: i64,
        max_seqlen_q: i64,
        max_seqlen_k: i64,
        window_left: i32,
        softmax_scale: f32,
        dtype: c_int,
        stream: HipStream,
    );

    /// flash_attn_varlen(.., causal = true) over contiguous K/V (prefill_attn, flash_attn.rs:15-37).
    pub fn varlen_prefill_attention(
        out: *mut c_void,
        q: *const c_void,
        k: *const c_void,
        v: *const c_void,
        cu_seqlens_q: *const u32,
        cu_seqlens_k: *const u32,
        total_k: i64,
        batch: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        max_seqlen_q: i64,
        max_seqlen_k: i64,
        window_left: i32,
        softmax_scale: f32,
        dtype: c_int,
        stream: HipStream,
    );

    /// Qwen3Attention::forward's prologue (qwen3.rs:161-199): q/k RMSNorm, RoPE and the KV append, one launch.
    pub fn qk_norm_rope_and_cache(
        q_out: *mut c_void,
        k_out: *mut c_void,
        qkv: *const c_void,
        qkv_row_stride: i64,
        q_norm_weight: *const c_void,
        k_norm_weight: *const c_void,
        eps: f64,
        cos_sin_cache: *const f32,
        max_position: i64,
        positions: *const i32,
        key_cache: *mut c_void,
        value_cache: *mut c_void,
        slot_mapping: *const i64,
        num_tokens: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        dtype: c_int,
        stream: HipStream,
    );

    /// Host: RotaryEmbedding's fp32 cos/sin table (crates/vllm-oxide/src/layers/rope.rs:50-83).
    pub fn oxide_rope_cos_sin_cache(
        cache: *mut f32,
        max_position: i64,
        rotary_dim: i64,
        base: f32,
    ) -> c_int;

    /// cu_seqlens_k and the decode slot mapping built on the device from context lengths and the table.
    pub fn build_decode_metadata_device(
        context_lens: *const u32,
        block_table: *const i32,
        max_blocks_per_seq: i64,
        batch: i64,
        block_size: i64,
        cu_seqlens_k: *mut u32,
        slot_mapping: *mut i64,
        stream: HipStream,
    );

    /// Allocation-free decode (graph capture, serving loops): partials in a 48 MiB static device
    /// array per GPU; larger shapes fail with OXIDE_ERR_SCRATCH_TOO_SMALL; overlapping calls on one GPU race.
    pub fn paged_decode_attention_noalloc(
        out: *mut c_void,
        q: *const c_void,
        key: *const c_void,
        value: *const c_void,
        slot_mapping: *const i64,
        k_cache: *mut c_void,
        v_cache: *mut c_void,
        cu_seqlens_k: *const u32,
        block_table: *const i32,
        max_blocks_per_seq: i64,
        num_blocks: i64,
        batch: i64,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        page_block_size: i64,
        max_seqlen_k: i64,
        window_left: i32,
        softmax_scale: f32,
        dtype: c_int,
        stream: HipStream,
    );

    /// First error recorded on the calling host thread since oxide_clear_error (OXIDE_OK = none).
    pub fn oxide_last_error() -> c_int;

    pub fn oxide_clear_error();

    /// Static description of an error code.
    pub fn oxide_error_string(
        code: c_int,
    ) -> *const c_char;

    /// Host: seeded counter-based N(0, 1) data (bit-identical for any thread count); 0 or 1 (bad argument).
    pub fn oxide_fill_normal(
        dst: *mut c_void,
        n: i64,
        seed: u64,
        /// the generator's stream id (one independent sequence per id), not a HIP stream
        stream: u64,
        dtype: c_int,
        threads: c_int,
    ) -> c_int;
}

/// The calling thread's pending library error, cleared on read: `Ok(())` or the code.
///
/// # Safety
/// Calls into the C library (no pointers are passed).
pub unsafe fn take_error() -> Result<(), c_int> {
    let code = oxide_last_error();
    if code == OXIDE_OK {
        Ok(())
    } else {
        oxide_clear_error();
        Err(code)
    }
}
