"""Synthetic decode-step workloads of the five benchmark configurations.

Host-side integer metadata only (numpy, seeded): context lengths, block tables,
the append slot of each sequence's new token, cu_seqlens_k.  The semantics are
those of the reference's decode step (crates/vllm-oxide/src/engine/mod.rs:232-278):
  * the new token's position is L - 1 and context_len = L includes it (:250-252);
  * its slot is compute_slot_mapping(seq, L - 1, 1) (kv_cache_manager.rs:115-135);
  * block-table rows hold ceil(L / block_size) block ids (sequence.rs num_blocks)
    and are padded with 0 to [B, max_blocks] (flash_attn.rs:74-86);
  * cu_seqlens_k = prefix sums of context_lens (metadata.rs:20-47).
Block ids are drawn without replacement from a seeded permutation of the pool.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

BLOCK_SIZE = 256  # crates/vllm-oxide/src/engine/sequence.rs:20


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    batch: int
    ctx_lo: int
    ctx_hi: int
    pool_blocks: int  # 0 = sized to fit the batch (sum of ceil(L/BS)) plus slack
    block_size: int = BLOCK_SIZE
    window_left: int = -1
    layers: int = 1
    shared_prefix: int = 0  # tokens of a prefix shared by every sequence (cfg4)
    dtype: str = "bf16"


CONFIGS = {
    1: DecodeConfig("cfg1-qwen3-0.6b-cpu-plumbing", 16, 8, 128, 4, 300, 1000, 64),
    2: DecodeConfig("cfg2-qwen3-0.6b-b32-28layers", 16, 8, 128, 32, 512, 4096, 4096, layers=28),
    3: DecodeConfig("cfg3-qwen3-8b-b64-ctx2k-8k", 32, 8, 128, 64, 2048, 8192, 8192),
    4: DecodeConfig("cfg4-qwen3-8b-prefix4096-w4096", 32, 8, 128, 128, 4096 + 64, 4096 + 1024, 8192,
                    window_left=4096, shared_prefix=4096),
    5: DecodeConfig("cfg5-qwen3-32b-b16-ctx32k-128k", 64, 8, 128, 16, 32768, 131072, 0),
}


@dataclass
class DecodeStep:
    cfg: DecodeConfig
    context_lens: np.ndarray      # uint32 [B], includes the appended token
    block_rows: list              # ragged int32 rows
    block_table: np.ndarray       # int32 [B, max_blocks], padded with 0
    slot_mapping: np.ndarray      # int64 [B], slot of each sequence's new token
    cu_seqlens_k: np.ndarray      # uint32 [B + 1]
    pool_blocks: int
    cow_pairs: np.ndarray = field(default_factory=lambda: np.zeros((0, 2), np.int64))

    @property
    def max_seqlen_k(self) -> int:
        return int(self.context_lens.max()) if self.context_lens.size else 0

    def kv_read_bytes(self, elem: int = 2) -> int:
        """Algorithmic K+V bytes the attention reads (window-limited)."""
        c = self.cfg
        L = self.context_lens.astype(np.int64)
        eff = np.minimum(L, c.window_left + 1) if c.window_left >= 0 else L
        return int(2 * eff.sum() * c.num_kv_heads * c.head_dim * elem)

    def unique_kv_read_bytes(self, elem: int = 2) -> int:
        """K+V bytes of the distinct cache rows the batch attends (window-limited): a
        row that several sequences reach through a shared block counts once.  Equal
        to kv_read_bytes() when no block is shared."""
        c = self.cfg
        L = self.context_lens.astype(np.int64)
        lo = np.maximum(L - 1 - c.window_left, 0) if c.window_left >= 0 else np.zeros_like(L)
        slots = [np.asarray(self.block_rows[b], np.int64)[np.arange(lo[b], L[b]) // c.block_size] * c.block_size
                 + np.arange(lo[b], L[b]) % c.block_size for b in range(len(L))]
        n = np.unique(np.concatenate(slots)).size if slots else 0
        return int(2 * n * c.num_kv_heads * c.head_dim * elem)

    def attn_unique_bytes(self, elem: int = 2) -> int:
        """attn_bytes() with the K+V rows counted once per distinct cache row: the
        least HBM traffic of a call that reads each shared row once."""
        return self.attn_bytes(elem) - self.kv_read_bytes(elem) + self.unique_kv_read_bytes(elem)

    def attn_bytes(self, elem: int = 2) -> int:
        """Algorithmic bytes of one decode-attention call: K+V read, q read, out
        written, block-table entries and seqlens read."""
        c = self.cfg
        L = self.context_lens.astype(np.int64)
        lo = np.maximum(L - 1 - c.window_left, 0) if c.window_left >= 0 else np.zeros_like(L)
        pages = (L + c.block_size - 1) // c.block_size - lo // c.block_size
        qo = 2 * c.batch * c.num_heads * c.head_dim * elem
        return self.kv_read_bytes(elem) + qo + int(4 * pages.sum()) + 4 * (c.batch + 1)

    def append_bytes(self, elem: int = 2) -> int:
        """Algorithmic bytes of the append: read K,V rows, write them, read slots."""
        c = self.cfg
        return c.batch * (4 * c.num_kv_heads * c.head_dim * elem + 8)


def make_decode_step(cfg: DecodeConfig, seed: int = 0, batch: int | None = None) -> DecodeStep:
    rng = np.random.default_rng(seed)
    B = cfg.batch if batch is None else batch
    BS = cfg.block_size
    L = rng.integers(cfg.ctx_lo, cfg.ctx_hi, size=B, endpoint=True).astype(np.int64)
    nblk = (L + BS - 1) // BS
    cow = np.zeros((0, 2), np.int64)
    if cfg.shared_prefix:
        assert cfg.shared_prefix % BS == 0
        n_shared = cfg.shared_prefix // BS
        # Every sequence gets a private copy of the last shared block (CoW) plus
        # its own suffix blocks.
        need = n_shared + int((nblk - n_shared + 1).sum())
        pool = cfg.pool_blocks or need + 64
        assert need <= pool, (need, pool)
        perm = rng.permutation(pool).astype(np.int32)
        shared = perm[:n_shared]
        pos = n_shared
        rows, pairs = [], []
        for b in range(B):
            own = perm[pos:pos + nblk[b] - n_shared + 1]
            pos += nblk[b] - n_shared + 1
            rows.append(np.concatenate([shared[:-1], own]).astype(np.int32))
            pairs.append((int(shared[-1]), int(own[0])))
        cow = np.array(pairs, dtype=np.int64)
    else:
        need = int(nblk.sum())
        pool = cfg.pool_blocks or need + 64
        assert need <= pool, (need, pool)
        perm = rng.permutation(pool).astype(np.int32)
        rows, pos = [], 0
        for b in range(B):
            rows.append(perm[pos:pos + nblk[b]])
            pos += nblk[b]
    width = int(nblk.max())
    table = np.zeros((B, width), dtype=np.int32)
    for b, r in enumerate(rows):
        table[b, :len(r)] = r
    pos_new = L - 1
    slots = np.array([int(rows[b][pos_new[b] // BS]) * BS + int(pos_new[b] % BS) for b in range(B)],
                     dtype=np.int64)
    cu = np.zeros(B + 1, dtype=np.uint32)
    cu[1:] = np.cumsum(L).astype(np.uint32)
    return DecodeStep(cfg, L.astype(np.uint32), rows, table, slots, cu, pool, cow)


def fill_normal(shape, seed: int, stream: int, dtype: str = "bf16", threads: int = 0) -> np.ndarray:
    """Seeded N(0, 1) host data from the library's counter-based generator
    (oxide_fill_normal): uint16 bit patterns for bf16 / f16, float32 for f32.  The same
    (seed, stream, shape) always gives the same bytes, whatever the thread count."""
    from . import _lib

    code = {"f16": 0, "bf16": 1, "f32": 2}[dtype]
    out = np.empty(shape, dtype=np.float32 if code == 2 else np.uint16)
    rc = _lib.load().oxide_fill_normal(out.ctypes.data, out.size, seed, stream, code, threads)
    if rc != 0:
        raise _lib.OxideError(f"oxide_fill_normal: error {rc}")
    return out
