"""GPU parity of KV append (reshape_and_cache), copy_blocks and gather_blocks.

All three are bitwise copies, so the bar is bit-exact equality with the oracle
(oracle/oxide_oracle.c, restating reshape_and_cache.cu:6-28 and copy_blocks.cu:8-28)
on identical seeded inputs.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from helpers import normal_bits, to_bits, to_torch

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def _ops():
    import oxide_paged_kv

    return oxide_paged_kv


def test_reshape_and_cache_reference_known_answer(device):
    """attention/mod.rs:161-230: arange K, 1000+arange V, slots [0,256,512] land
    at k[0,0], k[1,0], v[2,0] with max-diff 0."""
    import torch

    ka = GOLDEN["reshape_and_cache_known_answer"]
    H, D, T, NB, BS = ka["num_kv_heads"], ka["head_dim"], ka["num_tokens"], ka["num_blocks"], ka["block_size"]
    # PagedKVCache::new(1, 4, 256, 2, 64, BF16) -> [2, 1, 4, 256, 2, 64] zeros.
    buf = torch.zeros((2, 1, NB, BS, H, D), dtype=torch.bfloat16, device=device)
    kc, vc = buf[0, 0], buf[1, 0]
    key = torch.arange(0, T * H * D, dtype=torch.float32, device=device).reshape(T, H, D).bfloat16()
    val = torch.arange(1000, 1000 + T * H * D, dtype=torch.float32, device=device).reshape(T, H, D).bfloat16()
    sm = torch.tensor(ka["slot_mapping"], dtype=torch.int64, device=device)
    _ops().reshape_and_cache(key, val, kc, vc, sm)
    torch.cuda.synchronize()
    for cache, blk, off, src, t in ka["checks"]:
        got = (kc if cache == "k" else vc)[blk, off].float()
        want = (key if src == "key" else val)[t].float()
        assert float((got - want).abs().max()) == ka["max_diff"]
    # Every other slot is still zero.
    mask = torch.ones((NB, BS), dtype=torch.bool, device=device)
    mask[0, 0] = mask[1, 0] = mask[2, 0] = False
    assert not kc[mask].any() and not vc[mask].any()


@pytest.mark.parametrize("dtype,torch_dt,H,D", [
    ("bf16", "bfloat16", 8, 128),  # Qwen3 shape: 2 KiB rows, 128-bit path
    ("f16", "float16", 4, 64),
    ("f32", "float32", 2, 64),
    ("bf16", "bfloat16", 3, 5),    # 30-byte rows: per-element path
    ("f32", "float32", 1, 3),
])
def test_reshape_and_cache_random_vs_oracle(device, dtype, torch_dt, H, D):
    import torch

    rng = np.random.default_rng(1)
    NB, BS, T = 6, 32, 57
    esz = 4 if dtype == "f32" else 2
    raw = np.uint32 if esz == 4 else np.uint16
    kc = rng.integers(0, 2**(8 * esz), size=(NB, BS, H, D), dtype=np.uint64).astype(raw)
    vc = rng.integers(0, 2**(8 * esz), size=(NB, BS, H, D), dtype=np.uint64).astype(raw)
    key = rng.integers(0, 2**(8 * esz), size=(T, H, D), dtype=np.uint64).astype(raw)
    val = rng.integers(0, 2**(8 * esz), size=(T, H, D), dtype=np.uint64).astype(raw)
    slots = rng.choice(NB * BS, size=T, replace=False).astype(np.int64)
    slots[::7] = -1
    tdt = getattr(torch, torch_dt)
    ints = torch.int32 if esz == 4 else torch.int16
    sint = np.int32 if esz == 4 else np.int16

    def dev(a):
        return torch.from_numpy(a.view(sint)).to(device).view(tdt)

    gk, gv = dev(kc.copy()), dev(vc.copy())
    _ops().reshape_and_cache(dev(key), dev(val), gk, gv, torch.from_numpy(slots).to(device))
    oracle.reshape_and_cache(key, val, kc, vc, slots)
    torch.cuda.synchronize()
    assert np.array_equal(gk.view(ints).cpu().numpy().view(raw), kc)
    assert np.array_equal(gv.view(ints).cpu().numpy().view(raw), vc)


def test_reshape_and_cache_empty_and_errors(device):
    import torch

    ops = _ops()
    kc = torch.zeros((2, 16, 2, 8), dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    e = torch.empty((0, 2, 8), dtype=torch.bfloat16, device=device)
    ops.reshape_and_cache(e, e, kc, vc, torch.empty(0, dtype=torch.int64, device=device))
    assert not kc.any()
    with pytest.raises(ops.OxideError):
        ops.reshape_and_cache(e.double(), e.double(), kc.double(), vc.double(),
                              torch.empty(0, dtype=torch.int64, device=device))


def test_reshape_and_cache_decode_step_cfg3(device):
    """Full cfg3 decode append: 64 tokens into an 8192-block pool, bit-exact."""
    import torch
    from oxide_paged_kv.workload import CONFIGS, make_decode_step

    st = make_decode_step(CONFIGS[3], seed=3)
    c = st.cfg
    g = torch.Generator(device=device).manual_seed(3)
    kc = torch.randn((st.pool_blocks, c.block_size, c.num_kv_heads, c.head_dim), generator=g,
                     device=device, dtype=torch.float32).bfloat16()
    vc = torch.randn_like(kc, dtype=torch.float32).bfloat16()
    key = torch.randn((c.batch, c.num_kv_heads, c.head_dim), generator=g, device=device).bfloat16()
    val = torch.randn_like(key, dtype=torch.float32).bfloat16()
    kc0, vc0 = kc.clone(), vc.clone()
    sm = torch.from_numpy(st.slot_mapping).to(device)
    _ops().reshape_and_cache(key, val, kc, vc, sm)
    # torch index_put as the independent expectation.
    kc0.view(-1, c.num_kv_heads, c.head_dim)[sm] = key
    vc0.view(-1, c.num_kv_heads, c.head_dim)[sm] = val
    torch.cuda.synchronize()
    assert torch.equal(kc.view(torch.int16), kc0.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), vc0.view(torch.int16))


@pytest.mark.parametrize("shape,dtype", [((12, 256, 8, 128), "bf16"), ((9, 16, 3, 7), "f16"),
                                         ((5, 32, 2, 64), "f32")])
def test_copy_blocks_vs_oracle(device, shape, dtype):
    import torch

    rng = np.random.default_rng(2)
    esz = 4 if dtype == "f32" else 2
    raw, sint = (np.uint32, np.int32) if esz == 4 else (np.uint16, np.int16)
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    tint = torch.int32 if esz == 4 else torch.int16
    kc = rng.integers(0, 2**(8 * esz), size=shape, dtype=np.uint64).astype(raw)
    vc = rng.integers(0, 2**(8 * esz), size=shape, dtype=np.uint64).astype(raw)
    NB = shape[0]
    src_dst = rng.permutation(NB)
    npairs = NB // 2
    mapping = np.stack([src_dst[:npairs], src_dst[npairs:2 * npairs]], axis=1).astype(np.int64)
    gk = torch.from_numpy(kc.view(sint).copy()).to(device).view(tdt)
    gv = torch.from_numpy(vc.view(sint).copy()).to(device).view(tdt)
    _ops().copy_blocks(gk, gv, torch.from_numpy(mapping).to(device))
    oracle.copy_blocks(kc, vc, mapping)
    torch.cuda.synchronize()
    assert np.array_equal(gk.view(tint).cpu().numpy().view(raw), kc)
    assert np.array_equal(gv.view(tint).cpu().numpy().view(raw), vc)


@pytest.mark.parametrize("npairs", [65535, 70001])
def test_copy_blocks_many_pairs(device, npairs):
    """Up to 65535 pairs the launch puts a pair's slices along the grid's x and the
    pairs along y; beyond that (y is limited to 65535) pairs go along x.  Both
    orders, bit-exact against the oracle (small 128-byte blocks)."""
    import torch

    rng = np.random.default_rng(npairs)
    shape = (2 * npairs + 3, 8, 1, 8)
    kc = rng.integers(0, 2**16, size=shape, dtype=np.uint64).astype(np.uint16)
    vc = rng.integers(0, 2**16, size=shape, dtype=np.uint64).astype(np.uint16)
    perm = rng.permutation(shape[0])
    mapping = np.stack([perm[:npairs], perm[npairs:2 * npairs]], axis=1).astype(np.int64)
    gk = torch.from_numpy(kc.view(np.int16).copy()).to(device).view(torch.bfloat16)
    gv = torch.from_numpy(vc.view(np.int16).copy()).to(device).view(torch.bfloat16)
    _ops().copy_blocks(gk, gv, torch.from_numpy(mapping).to(device))
    oracle.copy_blocks(kc, vc, mapping)
    torch.cuda.synchronize()
    assert np.array_equal(gk.view(torch.int16).cpu().numpy().view(np.uint16), kc)
    assert np.array_equal(gv.view(torch.int16).cpu().numpy().view(np.uint16), vc)


def test_copy_blocks_src_equals_dst_is_identity(device):
    import torch

    g = torch.Generator(device=device).manual_seed(4)
    kc = torch.randn((4, 256, 8, 128), generator=g, device=device).bfloat16()
    vc = torch.randn_like(kc, dtype=torch.float32).bfloat16()
    k0, v0 = kc.clone(), vc.clone()
    _ops().copy_blocks(kc, vc, torch.tensor([[1, 1], [3, 3]], dtype=torch.int64, device=device))
    torch.cuda.synchronize()
    assert torch.equal(kc.view(torch.int16), k0.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), v0.view(torch.int16))


def test_copy_blocks_cfg4_cow(device):
    """cfg4: 128 copy-on-write pairs of 512 KiB blocks (Qwen3-8B shape), bit-exact."""
    import torch
    from oxide_paged_kv.workload import CONFIGS, make_decode_step

    st = make_decode_step(CONFIGS[4], seed=4)
    c = st.cfg
    g = torch.Generator(device=device).manual_seed(4)
    kc = torch.randn((st.pool_blocks, c.block_size, c.num_kv_heads, c.head_dim), generator=g,
                     device=device).bfloat16()
    vc = torch.randn_like(kc, dtype=torch.float32).bfloat16()
    pairs = torch.from_numpy(st.cow_pairs).to(device)
    _ops().copy_blocks(kc, vc, pairs)
    torch.cuda.synchronize()
    src, dst = pairs[:, 0], pairs[:, 1]
    assert torch.equal(kc[dst].view(torch.int16), kc[src].view(torch.int16))
    assert torch.equal(vc[dst].view(torch.int16), vc[src].view(torch.int16))


@pytest.mark.parametrize("with_v", [True, False])
def test_gather_blocks_vs_oracle(device, with_v):
    import torch

    rng = np.random.default_rng(5)
    kc = normal_bits(rng, (10, 256, 8, 128))
    vc = normal_bits(rng, (10, 256, 8, 128))
    ids = rng.choice(10, size=6, replace=False).astype(np.int32)
    gk, gv = _ops().gather_blocks(to_torch(kc, "bf16", device), to_torch(vc, "bf16", device) if with_v else None,
                                  torch.from_numpy(ids).to(device))
    ok, ov = oracle.gather_blocks(kc, vc if with_v else None, ids)
    assert np.array_equal(to_bits(gk).reshape(ok.shape), ok)
    if with_v:
        assert np.array_equal(to_bits(gv).reshape(ov.shape), ov)
    else:
        assert gv is None
