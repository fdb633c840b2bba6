"""Long-context decode parity that a lost or doubled key range cannot pass.

With N(0,1) data the attention output of a long sequence is an average over
many keys and shrinks like sqrt(e / n) (about 0.015 at 131k keys), so a kernel
that drops or double-counts one of the ~26 pieces a 131k sequence is cut into
stays inside the absolute tolerance.  These tests make the answer O(1) and
sensitive to every piece:

* needles: in each (sequence, kv head) a handful of keys point along the group's
  query direction with slightly different strengths, so their scores exceed
  every other key's by more than 35 (weight below e^-35 each for the rest).  They sit on the
  key boundaries of every first pass -- the first and last key, both sides of a
  stream-range boundary, of a 1024-key split and of a 256-key block, and the
  new token of the fused append -- so each lands in a different piece.  The
  expected output is the softmax over the needles alone, computed in fp64 from
  the bf16 values: a closed form that needs no oracle.  A lost piece removes a
  needle's V row, a doubled one doubles its weight; both move the output by
  O(0.1), far outside the bar.
* peaked softmax: q scaled by 8 on random data, so a few keys dominate and the
  output is O(1); checked against the oracle on sampled sequences.

Bars: the target's tolerance (max-abs 2e-2, max-rel 1e-2) and an error bar
scaled to each (sequence, head) row, max|got - want| <= 2e-2 max|want| + 1 bf16
ulp; the achieved errors are printed.
"""
import math

import numpy as np
import pytest

import oracle
from helpers import assert_attn_close, assert_attn_scaled, to_bits, to_f32

pytestmark = pytest.mark.gpu

PATHS = {1: "split", 2: "persistent", 3: "stream", 4: "rows"}


def _config(cfg_id):
    from oxide_paged_kv.workload import CONFIGS, DecodeConfig

    if cfg_id in CONFIGS:
        return CONFIGS[cfg_id]
    # Small batches that the shape policy gives 128-key splits (grids of fewer than 2048
    # 256-key workgroups), without and with a window.
    return {"b4-w300": DecodeConfig("b4-ctx0.3k-1k-w300", 32, 8, 128, 4, 300, 1000, 64, window_left=300),
            "b8": DecodeConfig("b8-ctx1-3000", 32, 8, 128, 8, 1, 3000, 128)}[cfg_id]


def _inputs(cfg_id, seed, device):
    import torch
    from oxide_paged_kv.workload import make_decode_step

    st = make_decode_step(_config(cfg_id), seed=seed)
    c = st.cfg
    g = torch.Generator(device=device).manual_seed(seed)
    shape = (st.pool_blocks, c.block_size, c.num_kv_heads, c.head_dim)
    kc = torch.randn(shape, generator=g, device=device).bfloat16()
    vc = torch.randn(shape, generator=g, device=device).bfloat16()
    return st, kc, vc, g


def _stream_range_starts(st, device):
    """Per sequence, the attended-key offsets (from the window start) at which a
    stream-pass key range begins: ranges cut the batch's attended keys laid end to
    end into CUs (rounded down to a multiple of 8) x 8 / Hkv equal parts."""
    import torch

    c = st.cfg
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    U = (cus - cus % 8) * (8 // c.num_kv_heads)
    L = st.context_lens.astype(np.int64)
    lo = np.maximum(L - 1 - c.window_left, 0) if c.window_left >= 0 else np.zeros_like(L)
    n = L - lo
    cu = np.concatenate([[0], np.cumsum(n)])
    K = int(cu[-1])
    starts = np.array([u * K // U for u in range(1, U)], np.int64)
    return [(starts[(starts > cu[b]) & (starts < cu[b + 1])] - cu[b] + lo[b]) for b in range(len(L))], lo


def _needle_positions(st, device, rng):
    """Up to 13 distinct key positions per sequence inside its attended keys."""
    starts, lo = _stream_range_starts(st, device)
    out = []
    for b, L in enumerate(st.context_lens.astype(np.int64)):
        a = int(lo[b])
        pos = {a, int(L) - 1}
        if len(starts[b]):
            x = int(rng.choice(starts[b]))
            pos |= {x - 1, x}
        for step in (1024, 512, 256, 128):
            m = [k for k in range(((a + step) // step) * step, int(L) - 1, step)]
            if m:
                x = int(rng.choice(m))
                pos |= {x - 1, x}
        pos.add(int(rng.integers(a, L)))
        out.append(sorted(p for p in pos if a <= p < L))
    return out


def _plant_needles(st, kc, vc, g, rng, device):
    """Queries and needles: per (sequence, kv head) a direction u; the group's queries
    are u plus N(0, 0.3^2) noise and needle i is lam_i * u, lam_i in [3.9, 4.0] (so the
    needles' weights are within 3x of each other).  Needles whose physical row another
    sequence already holds (a shared prefix block) are dropped.  Returns q, the new
    token's K/V rows (its K a needle too), and per sequence the needle positions and
    (fp32) K and V rows [n, Hkv, D]."""
    import torch

    c = st.cfg
    B, H, D, G = c.batch, c.num_kv_heads, c.head_dim, c.num_heads // c.num_kv_heads
    u = torch.randn((B, H, D), generator=g, device=device)
    q = (u[:, :, None, :] + 0.3 * torch.randn((B, H, G, D), generator=g, device=device)).reshape(B, H * G, D)
    q = q.bfloat16()
    knew = torch.randn((B, H, D), generator=g, device=device).bfloat16()
    vnew = torch.randn((B, H, D), generator=g, device=device).bfloat16()
    positions = _needle_positions(st, device, rng)
    BS = c.block_size
    claimed = set()  # physical rows: shared prefix blocks (cfg4) must not get two sequences' needles
    needles = []
    for b, pos in enumerate(positions):
        rows = st.block_rows[b]
        last = int(st.context_lens[b]) - 1
        phys = [int(rows[p // BS]) * BS + p % BS for p in pos]
        pos = [p for p, r in zip(pos, phys) if r not in claimed]
        claimed.update(int(rows[p // BS]) * BS + p % BS for p in pos)
        lam = torch.linspace(3.9, 4.0, len(pos), device=device)[torch.randperm(len(pos), device=device)]
        krows = (lam[:, None, None] * u[b][None]).bfloat16()  # [n, H, D]
        # The new token (key L - 1) gets its needle through the append only: its
        # cache row keeps random data, so an append that does not land first loses it.
        cached = [i for i, p in enumerate(pos) if p != last]
        blk = torch.tensor([int(rows[pos[i] // BS]) for i in cached], device=device, dtype=torch.int64)
        off = torch.tensor([pos[i] % BS for i in cached], device=device, dtype=torch.int64)
        kc[blk, off] = krows[cached]
        vrows = torch.empty_like(krows)
        vrows[cached] = vc[blk, off]
        if pos[-1] == last:
            knew[b] = krows[-1]
            vrows[-1] = vnew[b]
        needles.append((pos, krows.float().cpu().numpy(), vrows.float().cpu().numpy()))
    return q, knew, vnew, needles


def _needle_want(st, q, needles):
    """Softmax over the needles only, in fp64 from the bf16 values."""
    c = st.cfg
    G = c.num_heads // c.num_kv_heads
    qf = q.float().cpu().numpy().astype(np.float64)
    want = np.zeros((c.batch, c.num_heads, c.head_dim))
    scale = 1 / math.sqrt(c.head_dim)
    for b, (pos, kr, vr) in enumerate(needles):
        for h in range(c.num_heads):
            kh = h // G
            s = scale * (kr[:, kh].astype(np.float64) @ qf[b, h])
            w = np.exp(s - s.max())
            want[b, h] = (w / w.sum()) @ vr[:, kh].astype(np.float64)
    return want


@pytest.mark.parametrize("cfg_id", [1, "b4-w300", "b8", 3, 4, 5])
def test_decode_needles_full_size(device, cfg_id):
    """Full-size cfg1, cfg3, cfg4 (window 4096) and cfg5, and two small batches whose
    shape policy takes 128-key splits (one windowed): needles on the piece boundaries of
    every first pass (128/256/512/1024-key splits and blocks, stream ranges); fused
    append (the new token is a needle) then plain attention, through each of the three
    passes."""
    import torch
    import oxide_paged_kv as ox

    seed = 90 + (cfg_id if isinstance(cfg_id, int) else len(cfg_id))
    st, kc0, vc0, g = _inputs(cfg_id, seed, device)
    c = st.cfg
    if not isinstance(cfg_id, int):
        assert ox.split_tokens(c.batch, c.num_kv_heads, st.max_seqlen_k) == 128
    rng = np.random.default_rng(seed)
    q, knew, vnew, needles = _plant_needles(st, kc0, vc0, g, rng, device)
    want = _needle_want(st, q, needles)
    print(f"cfg{cfg_id} needles per sequence: {[len(n[0]) for n in needles]}", flush=True)
    sm = torch.from_numpy(st.slot_mapping).to(device)
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device)
    bt = torch.from_numpy(st.block_table).to(device)
    w = None if c.window_left < 0 else c.window_left
    scale = 1 / math.sqrt(c.head_dim)
    for path, name in PATHS.items():
        kc, vc = kc0.clone(), vc0.clone()
        for fused in (True, False):
            print(f"cfg{cfg_id} {name} {'fused append' if fused else 'after append'}", flush=True)
            got = to_f32(ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale, w,
                                        append=(knew, vnew, sm) if fused else None, path=path))
            assert_attn_close(got, want)
            assert_attn_scaled(got, want, label=f"cfg{cfg_id} {name} fused={fused}")
        del kc, vc
        torch.cuda.empty_cache()


def test_decode_needles_detect_a_lost_piece(device):
    """The needle bar is sharp: the same cfg3 batch with one needle's key row moved
    off the query direction (as if its piece were lost) fails the bar by far."""
    import torch
    import oxide_paged_kv as ox

    st, kc, vc, g = _inputs(3, 93, device)
    c = st.cfg
    q, knew, vnew, needles = _plant_needles(st, kc, vc, g, np.random.default_rng(3), device)
    want = _needle_want(st, q, needles)
    b = 5
    pos = needles[b][0][1]
    kc[int(st.block_rows[b][pos // c.block_size]), pos % c.block_size] = 0
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device)
    bt = torch.from_numpy(st.block_table).to(device)
    got = to_f32(ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, 1 / math.sqrt(c.head_dim),
                                append=(knew, vnew, torch.from_numpy(st.slot_mapping).to(device))))
    others = [i for i in range(c.batch) if i != b]
    assert_attn_scaled(got[others], want[others], label="untouched sequences")
    err = np.abs(got[b] - want[b]).max()
    print(f"sequence {b} with a needle removed: max err {err:.3f}", flush=True)
    assert err > 0.05


@pytest.mark.parametrize("cfg_id", [3, 5])
def test_decode_peaked_softmax_full_size(device, cfg_id):
    """Full-size cfg3 / cfg5 with q scaled by 8: a few keys dominate and outputs are
    O(1); each pass against the oracle on the longest, shortest and one middle
    sequence."""
    import torch
    import oxide_paged_kv as ox

    st, kc, vc, g = _inputs(cfg_id, 80 + cfg_id, device)
    c = st.cfg
    q = (8 * torch.randn((c.batch, c.num_heads, c.head_dim), generator=g, device=device)).bfloat16()
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device)
    bt = torch.from_numpy(st.block_table).to(device)
    scale = 1 / math.sqrt(c.head_dim)
    lens = st.context_lens.astype(np.int64)
    samples = sorted({int(lens.argmax()), int(lens.argmin()), c.batch // 2})
    wants = {}
    for b in samples:
        ids = torch.from_numpy(np.asarray(st.block_rows[b], np.int64)).to(device)
        wants[b] = oracle.paged_decode_attention(
            to_bits(q[b:b + 1]), to_bits(kc[ids]), to_bits(vc[ids]), np.array([0, lens[b]], np.uint32),
            np.arange(len(ids), dtype=np.int32)[None], scale, -1, threads=16)
    for path, name in PATHS.items():
        print(f"cfg{cfg_id} peaked {name}", flush=True)
        got = to_f32(ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale, path=path))
        for b in samples:
            assert np.abs(wants[b]).max() > 0.3  # the softmax is peaked: O(1) outputs
            assert_attn_close(got[b:b + 1], wants[b])
            assert_attn_scaled(got[b:b + 1], wants[b], label=f"cfg{cfg_id} {name} seq {b} L={lens[b]}")
