"""GPU parity of paged decode attention (split-KV, GQA, window) against the oracle.

Tolerance (the target's, for bf16/f16 output vs an fp32-accumulated reference):
max-abs 2e-2 and max-rel 1e-2, checked by helpers.assert_attn_close.  The oracle
(oracle/oxide_oracle.c, fp32 accumulate) is itself pinned against numpy fp64 in
tests/test_oracle.py.
"""
import math
import numpy as np
import pytest

import oracle
from helpers import assert_attn_close, assert_attn_scaled, normal_bits, to_bits, to_f32, to_torch

pytestmark = pytest.mark.gpu


def _run(device, q, kc, vc, cu, table, max_seqlen, scale, window, dtype, path=0):
    import torch
    import oxide_paged_kv as ox

    out = ox.decode_attn(to_torch(q, dtype, device), to_torch(kc, dtype, device),
                         to_torch(vc, dtype, device),
                         torch.from_numpy(cu.view(np.int32)).to(device),
                         torch.from_numpy(np.ascontiguousarray(table, dtype=np.int32)).to(device),
                         max_seqlen, scale, None if window < 0 else window, kc.shape[1], path=path)
    torch.cuda.synchronize()
    return out


def _case(seed, B, Hq, Hkv, D, BS, NB, lens, dtype="bf16"):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int64)
    nblk = (lens + BS - 1) // BS
    assert nblk.sum() <= NB
    perm = rng.permutation(NB).astype(np.int32)
    width = max(int(nblk.max()), 1)
    table = np.zeros((B, width), np.int32)
    pos = 0
    for b in range(B):
        table[b, :nblk[b]] = perm[pos:pos + nblk[b]]
        pos += nblk[b]
    cu = np.zeros(B + 1, np.uint32)
    cu[1:] = np.cumsum(lens)
    q = normal_bits(rng, (B, Hq, D), dtype)
    kc = normal_bits(rng, (NB, BS, Hkv, D), dtype)
    vc = normal_bits(rng, (NB, BS, Hkv, D), dtype)
    return q, kc, vc, cu, table, int(lens.max())


CASES = [
    # (B, Hq, Hkv, D, BS, NB, lens, window, dtype)
    (4, 16, 8, 128, 256, 64, [300, 1000, 557, 999], -1, "bf16"),        # cfg1 shape
    (3, 32, 8, 128, 256, 40, [2048, 4097, 3000], -1, "bf16"),           # G=4 (Qwen3-8B)
    (2, 64, 8, 128, 256, 80, [9000, 513], -1, "bf16"),                  # G=8 (Qwen3-32B)
    (3, 8, 8, 128, 256, 20, [1, 255, 256], -1, "bf16"),                 # G=1, page edges
    (2, 4, 2, 64, 256, 20, [700, 33], -1, "f16"),                       # G=2, D=64, f16
    (2, 32, 2, 64, 32, 120, [1500, 77], -1, "bf16"),                    # G=16, BS=32
    (3, 16, 8, 128, 16, 400, [1000, 17, 16], -1, "f16"),                # BS=16
    (4, 32, 8, 128, 256, 64, [5000, 4097, 100, 4096], 4096, "bf16"),    # window 4096
    (3, 16, 8, 128, 256, 30, [2000, 700, 101], 100, "bf16"),            # window 100
    (2, 16, 8, 128, 256, 10, [600, 5], 0, "bf16"),                      # window 0: last key only
    (5, 16, 8, 128, 256, 20, [0, 10, 0, 1, 300], -1, "bf16"),           # empty sequences
    (3, 40, 8, 128, 256, 40, [3000, 257, 1200], -1, "bf16"),            # G=5 (Qwen3-14B heads)
    (2, 28, 4, 128, 16, 300, [2100, 77], 500, "bf16"),                  # G=7 (Qwen2.5-7B), window
    (2, 12, 4, 64, 256, 20, [900, 31], -1, "f16"),                      # G=3, D=64
    (2, 24, 4, 128, 256, 20, [1500, 256], -1, "bf16"),                  # G=6
    (3, 16, 8, 128, 256, 10, [3, 1, 2], -1, "bf16"),                    # fewer keys than stream ranges
    # Qwen3-8B heads (the row pass's shape) with small pages, f16, windows, empty sequences
    (5, 32, 8, 128, 16, 300, [0, 10, 0, 1, 300], -1, "f16"),
    (3, 32, 8, 128, 32, 200, [2000, 700, 101], 100, "bf16"),
    (2, 32, 8, 128, 256, 20, [600, 5], 0, "bf16"),
]


@pytest.fixture(params=[1, 2, 3, 4], ids=["split", "persistent", "stream", "rows"])
def decode_path(request):
    """Runs a test once per pass-1 path (split grid, persistent balanced pass,
    wave-level stream pass, whole-row pass -- the stream pass for shapes the row
    pass does not take)."""
    return request.param


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_decode_vs_oracle(device, case, decode_path):
    B, Hq, Hkv, D, BS, NB, lens, window, dtype = case
    q, kc, vc, cu, table, mx = _case(11, B, Hq, Hkv, D, BS, NB, lens, dtype)
    scale = 1.0 / math.sqrt(D)
    print(f"decode case B={B} Hq={Hq} Hkv={Hkv} D={D} BS={BS} lens={lens} window={window} {dtype} "
          f"path={decode_path}", flush=True)
    got = to_f32(_run(device, q, kc, vc, cu, table, mx, scale, window, dtype, path=decode_path))
    want = oracle.paged_decode_attention(q, kc, vc, cu, table, scale, window, dtype)
    assert_attn_close(got, want)
    for b, L in enumerate(lens):
        if L == 0:
            assert not got[b].any()


def _random_shapes(seed, n):
    """Seeded random shapes over what the fixed cases combine separately: kv heads
    1/2/3/4/8, groups 1-8 and 16, D 64/128, page sizes 16/32/256, bf16/f16, ragged
    lengths with empty and tiny sequences, windows; up to 60k keys per case."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        Hkv = int(rng.choice([1, 2, 3, 4, 8]))
        G = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 16]))
        D = int(rng.choice([64, 128]))
        BS = int(rng.choice([16, 32, 256]))
        dtype = str(rng.choice(["bf16", "f16"]))
        B = int(rng.integers(1, 81))
        lens = rng.integers(0, min(max(1, 60000 // B), 6000) + 1, B)
        if rng.random() < 0.3:
            lens[rng.integers(0, B)] = 0
        if rng.random() < 0.3:
            lens[:] = rng.integers(1, 40, B)
        if lens.max() == 0:
            lens[0] = 5
        window = -1 if rng.random() < 0.6 else int(rng.integers(0, 3000))
        out.append((B, G * Hkv, Hkv, D, BS, int(((lens + BS - 1) // BS).sum()) + 3, lens.tolist(), window, dtype))
    return out


@pytest.mark.parametrize("case", _random_shapes(2024, 30), ids=[f"r{i}" for i in range(30)])
def test_decode_random_shapes_vs_oracle(device, case, decode_path):
    B, Hq, Hkv, D, BS, NB, lens, window, dtype = case
    q, kc, vc, cu, table, mx = _case(21, B, Hq, Hkv, D, BS, NB, lens, dtype)
    scale = 1.0 / math.sqrt(D)
    print(f"decode random B={B} Hq={Hq} Hkv={Hkv} D={D} BS={BS} max={max(lens)} window={window} {dtype} "
          f"path={decode_path}", flush=True)
    got = to_f32(_run(device, q, kc, vc, cu, table, mx, scale, window, dtype, path=decode_path))
    assert_attn_close(got, oracle.paged_decode_attention(q, kc, vc, cu, table, scale, window, dtype))
    for b, L in enumerate(lens):
        if L == 0:
            assert not got[b].any()


def test_decode_reference_smoke_shape(device):
    """attention/mod.rs:277-323 flash_attn_decode_runs: ctx 32, 4 heads, 4 kv heads,
    D 64, one block of 256 -> shape [1, 4, 64], no NaN (and here also parity)."""
    q, kc, vc, cu, table, mx = _case(12, 1, 4, 4, 64, 256, 1, [32])
    out = _run(device, q, kc, vc, cu, table, mx, 1 / 8.0, -1, "bf16")
    assert tuple(out.shape) == (1, 4, 64)
    got = to_f32(out)
    assert not np.isnan(got).any()
    assert_attn_close(got, oracle.paged_decode_attention(q, kc, vc, cu, table, 1 / 8.0))


def test_decode_constant_v_closed_form(device):
    """V rows all equal -> every output row is that V row (any q, any window)."""
    q, kc, vc, cu, table, mx = _case(13, 3, 32, 8, 128, 256, 40, [3000, 257, 1])
    row = normal_bits(np.random.default_rng(0), (8, 128))
    vc[:] = row[None, None]
    out = to_f32(_run(device, q, kc, vc, cu, table, mx, 0.0883883, -1, "bf16"))
    want = np.repeat(oracle.bf16_bits_to_f32(row), 4, axis=0)
    for b in range(3):
        np.testing.assert_allclose(out[b], want, atol=1e-2, rtol=1e-2)


def test_decode_placement_invariance_bit_exact(device):
    """Moving the pages to other physical blocks (and re-pointing the table) must
    not change one output bit: the reduction order depends on logical positions only."""
    q, kc, vc, cu, table, mx = _case(14, 4, 32, 8, 128, 256, 64, [5000, 4097, 100, 4096])
    a = to_bits(_run(device, q, kc, vc, cu, table, mx, 0.0883883, -1, "bf16"))
    perm = np.random.default_rng(1).permutation(64)
    inv = np.argsort(perm)
    kc2, vc2 = kc[inv], vc[inv]  # block i moves to slot perm[i]
    table2 = perm[table].astype(np.int32)
    b = to_bits(_run(device, q, kc2, vc2, cu, table2, mx, 0.0883883, -1, "bf16"))
    assert np.array_equal(a, b)


def test_decode_window_at_least_len_equals_no_window(device):
    q, kc, vc, cu, table, mx = _case(15, 3, 16, 8, 128, 256, 30, [2000, 700, 101])
    a = to_bits(_run(device, q, kc, vc, cu, table, mx, 0.0883883, -1, "bf16"))
    b = to_bits(_run(device, q, kc, vc, cu, table, mx, 0.0883883, 5000, "bf16"))
    assert np.array_equal(a, b)


def test_decode_ignores_padding_and_stale_nan(device):
    """Slots past L in the last page and padded table entries (block 0) hold NaN;
    the output must not see them."""
    q, kc, vc, cu, table, mx = _case(16, 2, 16, 8, 128, 256, 12, [300, 20])
    nan = np.uint16(0x7FC0)
    used = set()
    for b, L in enumerate([300, 20]):
        nb = (L + 255) // 256
        used.update(table[b, :nb].tolist())
        last = table[b, nb - 1]
        kc[last, L % 256 or 256:] = nan
        vc[last, L % 256 or 256:] = nan
    for blk in range(12):
        if blk not in used:
            kc[blk] = nan
            vc[blk] = nan
    got = to_f32(_run(device, q, kc, vc, cu, table, mx, 0.0883883, -1, "bf16"))
    want = oracle.paged_decode_attention(q, kc, vc, cu, table, 0.0883883)
    assert_attn_close(got, want)


def test_decode_cfg3_full_size_sampled(device):
    """Full cfg3 (Qwen3-8B, B=64, ctx U[2048,8192], 8192-block pool): the whole batch
    runs on the GPU; 6 sampled sequences are checked against the oracle."""
    import torch
    import oxide_paged_kv as ox
    from oxide_paged_kv.workload import CONFIGS, make_decode_step

    st = make_decode_step(CONFIGS[3], seed=7)
    c = st.cfg
    g = torch.Generator(device=device).manual_seed(7)
    shape = (st.pool_blocks, c.block_size, c.num_kv_heads, c.head_dim)
    kc = torch.randn(shape, generator=g, device=device).bfloat16()
    vc = torch.randn(shape, generator=g, device=device).bfloat16()
    q = torch.randn((c.batch, c.num_heads, c.head_dim), generator=g, device=device).bfloat16()
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device)
    bt = torch.from_numpy(st.block_table).to(device)
    scale = 1 / math.sqrt(c.head_dim)
    out = to_f32(ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale))
    for b in [0, 9, 17, 31, 50, 63]:
        rows = st.block_rows[b]
        ids = torch.from_numpy(np.asarray(rows, np.int64)).to(device)
        kb, vb = to_bits(kc[ids]), to_bits(vc[ids])
        L = int(st.context_lens[b])
        want = oracle.paged_decode_attention(
            to_bits(q[b:b + 1]), kb, vb, np.array([0, L], np.uint32),
            np.arange(len(rows), dtype=np.int32)[None], scale)
        assert_attn_close(out[b:b + 1], want)


def test_decode_workspace_reuse_across_shapes(device):
    """One workspace serves several calls of different shapes (and holds the
    previous call's partials): each result must equal the same call made with a
    fresh workspace, bit for bit."""
    import torch
    import oxide_paged_kv as ox

    cases = [(4, 32, 8, 128, 256, 64, [5000, 4097, 100, 4096]), (3, 16, 8, 128, 256, 30, [2000, 700, 101]),
             (2, 64, 8, 128, 256, 80, [9000, 513])]
    ws = torch.full((64 << 20,), 0x7F, dtype=torch.uint8, device=device)
    for rep in range(2):
        for i, (B, Hq, Hkv, D, BS, NB, lens) in enumerate(cases):
            q, kc, vc, cu, table, mx = _case(20 + i, B, Hq, Hkv, D, BS, NB, lens)
            args = (to_torch(q, "bf16", device), to_torch(kc, "bf16", device), to_torch(vc, "bf16", device),
                    torch.from_numpy(cu.view(np.int32)).to(device), torch.from_numpy(table).to(device), mx,
                    0.0883883)
            shared = to_bits(ox.decode_attn(*args, workspace=ws))
            fresh = to_bits(ox.decode_attn(*args))
            torch.cuda.synchronize()
            assert np.array_equal(shared, fresh), (rep, i)


def _full_size_inputs(cfg_id, seed, device):
    import torch
    from oxide_paged_kv.workload import CONFIGS, make_decode_step

    st = make_decode_step(CONFIGS[cfg_id], seed=seed)
    c = st.cfg
    g = torch.Generator(device=device).manual_seed(seed)
    shape = (st.pool_blocks, c.block_size, c.num_kv_heads, c.head_dim)
    kc = torch.randn(shape, generator=g, device=device).bfloat16()
    vc = torch.randn(shape, generator=g, device=device).bfloat16()
    q = torch.randn((c.batch, c.num_heads, c.head_dim), generator=g, device=device).bfloat16()
    return st, kc, vc, q


def _check_sampled(st, kc, vc, q, out, samples, window=-1):
    """Oracle on the sampled sequences' own blocks (gathered to the host)."""
    import torch

    scale = 1 / math.sqrt(st.cfg.head_dim)
    for b in samples:
        rows = st.block_rows[b]
        ids = torch.from_numpy(np.asarray(rows, np.int64)).to(kc.device)
        kb, vb = to_bits(kc[ids]), to_bits(vc[ids])
        L = int(st.context_lens[b])
        want = oracle.paged_decode_attention(
            to_bits(q[b:b + 1]), kb, vb, np.array([0, L], np.uint32),
            np.arange(len(rows), dtype=np.int32)[None], scale, window, threads=16)
        assert_attn_close(out[b:b + 1], want)
        assert_attn_scaled(out[b:b + 1], want, label=f"seq {b} L={L}")


def test_decode_cfg4_prefix_cow_window_full_size(device):
    """cfg4 at full size: 128 sequences share a 4096-token prefix (16 blocks); the
    last shared block is copied per sequence with copy_blocks (copy-on-write), each
    sequence appends its new token, then decode attention with window 4096."""
    import torch
    import oxide_paged_kv as ox

    st, kc, vc, q = _full_size_inputs(4, 41, device)
    c = st.cfg
    print(f"cfg4 B={c.batch} pool={st.pool_blocks} cow_pairs={len(st.cow_pairs)}", flush=True)
    pairs = torch.from_numpy(st.cow_pairs).to(device)
    ox.copy_blocks(kc, vc, pairs)
    knew = torch.randn((c.batch, c.num_kv_heads, c.head_dim), device=device).bfloat16()
    vnew = torch.randn_like(knew, dtype=torch.float32).bfloat16()
    ox.reshape_and_cache(knew, vnew, kc, vc, torch.from_numpy(st.slot_mapping).to(device))
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device)
    bt = torch.from_numpy(st.block_table).to(device)
    out = to_f32(ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, 1 / math.sqrt(c.head_dim),
                                c.window_left))
    # CoW copies are bit-exact, and every sequence's private copy equals the shared block.
    src, dst = pairs[:, 0], pairs[:, 1]
    # (the appended tokens sit past the prefix, so the copies are still intact)
    assert torch.equal(kc[dst].view(torch.int16), kc[src].view(torch.int16))
    assert torch.equal(vc[dst].view(torch.int16), vc[src].view(torch.int16))
    _check_sampled(st, kc, vc, q, out, [0, 37, 127], c.window_left)


def test_decode_windowed_stream_repeats_bit_identical(device):
    """cfg4 at full size through the windowed stream pass, five calls in a row: the
    kernels are deterministic, so every call must give the first one's bits (the
    merge reads the attended-key prefix sums pass 1 publishes; a copy made before
    every thread had written its part once gave wrong pieces on some calls)."""
    import torch
    import oxide_paged_kv as ox

    st, kc, vc, q = _full_size_inputs(4, 43, device)
    c = st.cfg
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device)
    bt = torch.from_numpy(st.block_table).to(device)
    assert ox.split_tokens(c.batch, c.num_kv_heads, st.max_seqlen_k) == -1
    outs = [to_bits(ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, 1 / math.sqrt(c.head_dim), c.window_left))
            for _ in range(5)]
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    _check_sampled(st, kc, vc, q, to_f32(ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k,
                                                         1 / math.sqrt(c.head_dim), c.window_left)),
                   [1, 64, 126], c.window_left)


def test_decode_path_policy(device):
    """Shapes with >= ~1024 keys per stream range take the wave-level stream pass
    (split_tokens -1: cfg5, cfg3, cfg4), smaller ones a split grid (cfg2); kv head
    counts that do not divide 8 take the persistent pass when long (split_tokens 0)."""
    import oxide_paged_kv as ox

    assert ox.split_tokens(16, 8, 131072) == -1
    assert ox.split_tokens(64, 8, 8192) == -1
    assert ox.split_tokens(128, 8, 5120) == -1
    assert ox.split_tokens(32, 8, 4096) == 256
    assert ox.split_tokens(8, 8, 32768) == 512        # few long sequences: split grid
    assert ox.split_tokens(8, 8, 131072) == -1        # ... unless the ranges reach 4096 keys
    assert ox.split_tokens(16, 16, 131072) == 0
    assert ox.split_tokens(64, 8, 8192, path="split") == 1024
    assert ox.split_tokens(16, 8, 131072, path="split") == 1024
    assert ox.split_tokens(64, 8, 8192, path="persistent") == 0
    assert ox.split_tokens(64, 8, 8192, path="stream") == -1
    assert ox.split_tokens(16, 16, 131072, path="stream") == 0   # kv heads not dividing 8
    assert ox.split_tokens(64, 8, 8192) == -1
    # The row pass: only when forced, and only for its shape (else the stream pass).
    assert ox.split_tokens(64, 8, 8192, num_heads=32) == -1
    assert ox.split_tokens(64, 8, 8192, path="rows", num_heads=32) == -2
    assert ox.split_tokens(64, 8, 8192, path="rows", num_heads=32, page_block_size=48) == -1
    assert ox.split_tokens(64, 8, 8192, path="rows", num_heads=16) == -1
    assert ox.split_tokens(64, 8, 8192, path="rows", num_heads=32, head_dim=64) == -1
    assert ox.split_tokens(2000, 8, 8192, path="rows", num_heads=32) == -1  # beyond its LDS table
    assert ox.split_tokens(32, 8, 4096, num_heads=16) == 256


@pytest.mark.parametrize("cfg_id", [3, 4, 5])
def test_decode_paths_agree_full_size(device, cfg_id):
    """Full-size cfg3 / cfg4 (window 4096: the stream pass balances attended keys) /
    cfg5 through all three pass-1 paths: outputs agree within rounding of the partial
    merges (max-abs 2e-2, the attention tolerance)."""
    import torch
    import oxide_paged_kv as ox

    st, kc, vc, q = _full_size_inputs(cfg_id, 70 + cfg_id, device)
    c = st.cfg
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device)
    bt = torch.from_numpy(st.block_table).to(device)
    outs = []
    for path in (1, 2, 3, 4):
        print(f"cfg{cfg_id} path {path}", flush=True)
        outs.append(to_f32(ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, 1 / math.sqrt(c.head_dim),
                                          None if c.window_left < 0 else c.window_left, path=path)))
    assert_attn_close(outs[1], outs[0])
    assert_attn_close(outs[2], outs[0])
    assert_attn_scaled(outs[1], outs[0], label="persistent vs split")
    assert_attn_scaled(outs[2], outs[0], label="stream vs split")
    assert_attn_close(outs[3], outs[0])
    assert_attn_scaled(outs[3], outs[0], label="rows vs split")
    lens = st.context_lens.astype(np.int64)
    for o in outs[1:]:
        _check_sampled(st, kc, vc, q, o, [int(lens.argmax()), int(lens.argmin())], c.window_left)


def test_decode_cfg5_long_context_full_size(device):
    """cfg5 at full size: Qwen3-32B decode shape (G = 8), 16 sequences of 32k-128k
    keys; the longest and the shortest sequences are checked against the oracle."""
    import torch
    import oxide_paged_kv as ox

    st, kc, vc, q = _full_size_inputs(5, 51, device)
    c = st.cfg
    print(f"cfg5 B={c.batch} pool={st.pool_blocks} max_len={st.max_seqlen_k}", flush=True)
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device)
    bt = torch.from_numpy(st.block_table).to(device)
    out = to_f32(ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, 1 / math.sqrt(c.head_dim)))
    lens = st.context_lens.astype(np.int64)
    _check_sampled(st, kc, vc, q, out, [int(lens.argmax()), int(lens.argmin())])


@pytest.mark.parametrize("batch,ctx_hi,want_split", [(64, 4096, 512), (64, 8192, 1024), (16, 4096, 256),
                                                    (8, 3000, 128)])
def test_decode_each_split_size_sampled(device, batch, ctx_hi, want_split):
    """One batch per split size the split grid picks (128, 256, 512 and 1024 keys per
    workgroup; the split path is forced, the shape policy may prefer the stream
    pass), Qwen3-8B heads, sampled sequences checked against the oracle."""
    import torch
    import oxide_paged_kv as ox
    from oxide_paged_kv.workload import DecodeConfig, make_decode_step

    cfg = DecodeConfig(f"split{want_split}", 32, 8, 128, batch, 1, ctx_hi, 0)
    st = make_decode_step(cfg, seed=want_split)
    g = torch.Generator(device=device).manual_seed(want_split)
    shape = (st.pool_blocks, 256, 8, 128)
    kc = torch.randn(shape, generator=g, device=device).bfloat16()
    vc = torch.randn(shape, generator=g, device=device).bfloat16()
    q = torch.randn((batch, 32, 128), generator=g, device=device).bfloat16()
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device)
    bt = torch.from_numpy(st.block_table).to(device)
    assert ox.split_tokens(batch, 8, st.max_seqlen_k, path="split") == want_split
    out = to_f32(ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, 1 / math.sqrt(128), path="split"))
    lens = st.context_lens.astype(np.int64)
    _check_sampled(st, kc, vc, q, out, sorted({0, int(lens.argmax()), int(lens.argmin()), batch - 1}))


FUSED_CASES = [
    # (B, Hq, Hkv, D, BS, NB, lens, window, dtype)
    (4, 16, 8, 128, 256, 64, [300, 1000, 557, 999], -1, "bf16"),
    (3, 64, 8, 128, 256, 80, [9000, 513, 1], -1, "bf16"),
    (5, 16, 8, 128, 256, 20, [0, 10, 0, 1, 300], -1, "bf16"),
    (2, 4, 2, 64, 16, 200, [700, 33], 100, "f16"),
    (4, 32, 8, 128, 256, 64, [5000, 4097, 100, 4096], 4096, "bf16"),
]


@pytest.mark.parametrize("case", FUSED_CASES, ids=[f"f{i}" for i in range(len(FUSED_CASES))])
def test_decode_fused_append_equals_append_then_attend(device, case, decode_path):
    """paged_decode_attention_append == reshape_and_cache + paged_decode_attention,
    bit for bit (output and caches); slot -1 skips the append."""
    import torch
    import oxide_paged_kv as ox

    B, Hq, Hkv, D, BS, NB, lens, window, dtype = case
    q, kc, vc, cu, table, mx = _case(31, B, Hq, Hkv, D, BS, NB, lens, dtype)
    rng = np.random.default_rng(32)
    knew = normal_bits(rng, (B, Hkv, D), dtype)
    vnew = normal_bits(rng, (B, Hkv, D), dtype)
    used = {int(table[b, i]) for b, L in enumerate(lens) for i in range((L + BS - 1) // BS)}
    spare = [blk for blk in range(NB) if blk not in used]
    # Sequences with no keys append into distinct spare blocks (distinct slots: the
    # reference kernel's result is undefined when two tokens share a slot).
    slots = np.array([table[b, (L - 1) // BS] * BS + (L - 1) % BS if L > 0 else spare[b] * BS + 3
                      for b, L in enumerate(lens)], np.int64)
    slots[1 % B] = -1  # one sequence skips its append
    args = lambda k, v: (to_torch(q, dtype, device), k, v, torch.from_numpy(cu.view(np.int32)).to(device),
                         torch.from_numpy(table).to(device), mx, 1 / math.sqrt(D),
                         None if window < 0 else window, BS)
    k1, v1 = to_torch(kc, dtype, device), to_torch(vc, dtype, device)
    kn, vn, sm = to_torch(knew, dtype, device), to_torch(vnew, dtype, device), torch.from_numpy(slots).to(device)
    ox.reshape_and_cache(kn, vn, k1, v1, sm)
    want = to_bits(ox.decode_attn(*args(k1, v1), path=decode_path))
    k2, v2 = to_torch(kc, dtype, device), to_torch(vc, dtype, device)
    got = to_bits(ox.decode_attn(*args(k2, v2), append=(kn, vn, sm), path=decode_path))
    torch.cuda.synchronize()
    assert np.array_equal(got, want)
    assert np.array_equal(to_bits(k2), to_bits(k1))
    assert np.array_equal(to_bits(v2), to_bits(v1))


@pytest.mark.parametrize("cfg_id,path", [(3, 0), (4, 0), (5, 0), (3, 4), (4, 4)],
                         ids=["cfg3", "cfg4", "cfg5", "cfg3-rows", "cfg4-rows"])
def test_decode_fused_append_full_size(device, cfg_id, path):
    """Full-size cfg3 / cfg4 (window 4096) / cfg5 step: fused append + attention
    equals the two calls (by shape, and through the row pass)."""
    import torch
    import oxide_paged_kv as ox

    st, kc, vc, q = _full_size_inputs(cfg_id, 60 + cfg_id, device)
    c = st.cfg
    g = torch.Generator(device=device).manual_seed(cfg_id)
    kn = torch.randn((c.batch, c.num_kv_heads, c.head_dim), generator=g, device=device).bfloat16()
    vn = torch.randn((c.batch, c.num_kv_heads, c.head_dim), generator=g, device=device).bfloat16()
    sm = torch.from_numpy(st.slot_mapping).to(device)
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device)
    bt = torch.from_numpy(st.block_table).to(device)
    scale = 1 / math.sqrt(c.head_dim)
    k2, v2 = kc.clone(), vc.clone()
    ox.reshape_and_cache(kn, vn, kc, vc, sm)
    w = None if c.window_left < 0 else c.window_left
    want = ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale, w, path=path)
    got = ox.decode_attn(q, k2, v2, cu, bt, st.max_seqlen_k, scale, w, append=(kn, vn, sm), path=path)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(k2.view(torch.int16), kc.view(torch.int16))
    assert torch.equal(v2.view(torch.int16), vc.view(torch.int16))


def test_kernels_vs_committed_goldens(device):
    """Decode and prefill kernels against the committed fp64 goldens (small seeded
    cases, G 1/2/4/8, window none/100), within the attention tolerance."""
    import importlib.util
    from pathlib import Path

    import torch
    import oxide_paged_kv as ox

    here = Path(__file__).parent / "golden"
    gold = np.load(here / "attention_goldens.npz")
    spec = importlib.util.spec_from_file_location("gold", here / "make_attention_goldens.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    for i, sp in enumerate(mod.SPECS):
        q, kc, vc, cuq, cuk, table, scale = mod.case_inputs(sp)
        print(f"golden case{i} {sp[0]} G={sp[2]} window={sp[7]}", flush=True)
        t = lambda a: to_torch(a, "bf16", device)  # noqa: E731
        w = None if sp[7] < 0 else sp[7]
        if sp[0] == "decode":
            out = ox.decode_attn(t(q), t(kc), t(vc), torch.from_numpy(cuk.view(np.int32)).to(device),
                                 torch.from_numpy(table).to(device), int(np.diff(cuk).max()), scale, w, sp[4])
        else:
            out = ox.prefill_attn(t(q), t(kc), t(vc), torch.from_numpy(cuq.view(np.int32)).to(device),
                                  torch.from_numpy(cuk.view(np.int32)).to(device), int(np.diff(cuq).max()),
                                  int(np.diff(cuk).max()), scale, torch.from_numpy(table).to(device), w)
        torch.cuda.synchronize()
        assert_attn_close(to_f32(out), gold[f"case{i}"])


def test_decode_batch_beyond_stream_table(device):
    """4100 sequences (more than the stream pass's LDS table of sequence boundaries):
    the stream path, even when forced, falls back to the persistent pass, and every
    path matches the oracle on sampled sequences."""
    import torch
    import oxide_paged_kv as ox

    B, Hq, Hkv, D, BS = 4100, 8, 8, 64, 16
    rng = np.random.default_rng(41)
    lens = rng.integers(0, 40, B)
    q, kc, vc, cu, table, max_len = _case(41, B, Hq, Hkv, D, BS, int(((lens + BS - 1) // BS).sum()) + 4,
                                         lens, "bf16")
    assert ox.split_tokens(B, Hkv, max_len) != -1
    sample = [0, 1, 2, 1000, 2047, 4096, 4097, B - 1]
    want = oracle.paged_decode_attention(q[sample], kc, vc,
                                         np.concatenate([[0], np.cumsum(lens[sample])]).astype(np.uint32),
                                         table[sample], 0.125, -1, "bf16")
    for path in (0, 1, 2, 3):
        if path == 3:
            assert ox.split_tokens(B, Hkv, max_len, path=path) == 0
        print(f"batch {B} path {path}", flush=True)
        got = to_f32(_run(device, q, kc, vc, cu, table, max_len, 0.125, -1, "bf16", path=path))
        assert_attn_close(got[sample], want)
