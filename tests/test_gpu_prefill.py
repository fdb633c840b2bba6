"""GPU parity of prefill attention (paged and contiguous, causal, GQA, window) against
the oracle.

Tolerance (the target's, for bf16/f16 output vs an fp32-accumulated reference):
max-abs 2e-2 and max-rel 1e-2 (helpers.assert_attn_close).  The oracle's prefill
(oracle/oxide_oracle.c) is pinned in tests/test_oracle.py against a dense numpy fp64
routine, the decode oracle row by row, and a hand-worked FlashAttention 2 mask case.
"""
import math

import numpy as np
import pytest

import oracle
from helpers import assert_attn_close, normal_bits, to_f32, to_torch

pytestmark = pytest.mark.gpu


def _case(seed, lq, lk, Hq, Hkv, D, BS, dtype="bf16", spare=2):
    rng = np.random.default_rng(seed)
    lq = np.asarray(lq, np.int64)
    lk = np.asarray(lk, np.int64)
    B = len(lq)
    nblk = (lk + BS - 1) // BS
    NB = int(nblk.sum()) + spare
    perm = rng.permutation(NB).astype(np.int32)
    table = np.zeros((B, max(int(nblk.max()), 1)), np.int32)
    pos = 0
    for b in range(B):
        table[b, :nblk[b]] = perm[pos:pos + nblk[b]]
        pos += nblk[b]
    cuq = np.zeros(B + 1, np.uint32)
    cuq[1:] = np.cumsum(lq)
    cuk = np.zeros(B + 1, np.uint32)
    cuk[1:] = np.cumsum(lk)
    q = normal_bits(rng, (int(cuq[-1]), Hq, D), dtype)
    kc = normal_bits(rng, (NB, BS, Hkv, D), dtype)
    vc = normal_bits(rng, (NB, BS, Hkv, D), dtype)
    return q, kc, vc, cuq, cuk, table


def _contiguous(kc, cuk, table):
    NB, BS, Hkv, D = kc.shape
    rows = []
    for b in range(len(cuk) - 1):
        j = np.arange(int(cuk[b + 1] - cuk[b]))
        rows.append(table[b, j // BS].astype(np.int64) * BS + j % BS)
    rows = np.concatenate(rows) if rows else np.zeros(0, np.int64)
    return np.ascontiguousarray(kc.reshape(-1, Hkv, D)[rows])


def _gpu(device, q, k, v, cuq, cuk, table, scale, window, dtype, paged=True):
    import torch
    import oxide_paged_kv as ox

    t = lambda a: to_torch(a, dtype, device)  # noqa: E731
    mq = int(np.max(np.diff(cuq))) if len(cuq) > 1 else 0
    mk = int(np.max(np.diff(cuk))) if len(cuk) > 1 else 0
    out = ox.prefill_attn(t(q), t(k), t(v), torch.from_numpy(cuq.view(np.int32)).to(device),
                          torch.from_numpy(cuk.view(np.int32)).to(device), mq, mk, scale,
                          torch.from_numpy(table).to(device) if paged else None,
                          None if window < 0 else window)
    torch.cuda.synchronize()
    return out


CASES = [
    # (lq, lk, Hq, Hkv, D, BS, window, dtype)
    ([300, 77], [300, 77], 32, 8, 128, 256, -1, "bf16"),              # plain prompts, G=4
    ([128, 40, 200], [1000, 40, 457], 32, 8, 128, 256, -1, "bf16"),   # prefix hits (Lk > Lq)
    ([64, 9], [64, 4], 16, 8, 128, 16, -1, "bf16"),                   # Lk < Lq: leading rows see nothing
    ([0, 50, 0, 1], [10, 50, 0, 1], 16, 8, 128, 256, -1, "bf16"),     # empty query lists / keys
    ([513, 100], [513, 900], 16, 8, 128, 256, 100, "bf16"),           # window 100
    ([200], [1200], 64, 8, 128, 256, 4096, "bf16"),                   # G=8, window > context
    ([130, 70], [130, 270], 8, 8, 128, 32, -1, "f16"),                # G=1, f16, BS=32
    ([100, 33], [100, 66], 4, 2, 64, 16, 7, "bf16"),                  # G=2, D=64, window 7
    ([90], [300], 32, 2, 64, 256, -1, "f16"),                         # G=16, D=64
    ([40], [40], 24, 8, 128, 256, -1, "bf16"),                        # G=3 (rows not a power of 2)
    # No cached prefix and prompts of at most 2048 tokens: workgroups take row tiles in
    # pairs (n - 1 - i, then i), including an odd tile count's middle tile alone.
    ([70, 33], [70, 33], 32, 8, 128, 256, -1, "bf16"),                # 3 and 2 row tiles
    ([300, 150], [300, 150], 32, 8, 128, 64, 50, "f16"),              # window 50, BS=64
    ([2048], [2048], 16, 8, 64, 32, -1, "bf16"),                      # the longest paired prompt
]


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_prefill_paged_vs_oracle(device, case):
    lq, lk, Hq, Hkv, D, BS, window, dtype = case
    q, kc, vc, cuq, cuk, table = _case(21, lq, lk, Hq, Hkv, D, BS, dtype)
    scale = 1.0 / math.sqrt(D)
    print(f"prefill case lq={lq} lk={lk} Hq={Hq} Hkv={Hkv} D={D} BS={BS} w={window} {dtype}", flush=True)
    got = to_f32(_gpu(device, q, kc, vc, cuq, cuk, table, scale, window, dtype))
    want = oracle.prefill_attention(q, kc, vc, cuq, cuk, scale, table, window, dtype)
    assert_attn_close(got, want)
    # Rows that see no key are exactly zero.
    for b in range(len(lq)):
        for i in range(lq[b]):
            if i + lk[b] - lq[b] < 0:
                assert not got[int(cuq[b]) + i].any()


def _random_shapes(seed, n):
    """Seeded random shapes: 1-3 prompts of up to 300 new tokens behind up to 500
    cached keys (or fewer keys than queries), kv heads 1/2/4/8, groups 1-8 and 16,
    D 64/128, page sizes 16/32/64/256 (per-row and per-tile block lookups), windows,
    bf16/f16; at most ~1e9 multiply-adds per case for the oracle."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        B = int(rng.integers(1, 4))
        Hkv = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 16]))
        D = int(rng.choice([64, 128]))
        lq = rng.integers(0, 301, B)
        pre = rng.integers(0, 501, B) if rng.random() < 0.7 else -rng.integers(0, 50, B)
        lk = np.maximum(lq + pre, 0)
        if lq.sum() == 0 or lk.sum() == 0:
            continue
        if int((lq * lk).sum()) * G * Hkv * D > 1e9:
            continue
        window = -1 if rng.random() < 0.6 else int(rng.integers(0, 600))
        out.append((lq.tolist(), lk.tolist(), G * Hkv, Hkv, D, int(rng.choice([16, 32, 64, 256])), window,
                    str(rng.choice(["bf16", "f16"]))))
    return out


@pytest.mark.parametrize("case", _random_shapes(77, 24), ids=[f"r{i}" for i in range(24)])
def test_prefill_random_shapes_vs_oracle(device, case):
    lq, lk, Hq, Hkv, D, BS, window, dtype = case
    q, kc, vc, cuq, cuk, table = _case(31, lq, lk, Hq, Hkv, D, BS, dtype)
    scale = 1.0 / math.sqrt(D)
    print(f"prefill random lq={lq} lk={lk} Hq={Hq} Hkv={Hkv} D={D} BS={BS} w={window} {dtype}", flush=True)
    got = to_f32(_gpu(device, q, kc, vc, cuq, cuk, table, scale, window, dtype))
    assert_attn_close(got, oracle.prefill_attention(q, kc, vc, cuq, cuk, scale, table, window, dtype))


@pytest.mark.parametrize("case", [CASES[1], CASES[4], CASES[7]], ids=["prefix", "window", "d64"])
def test_prefill_contiguous_equals_paged(device, case):
    """flash_attn_varlen form (contiguous K/V): same kernel, so bit-identical to the paged
    form over the same keys, and within tolerance of the oracle."""
    import torch

    lq, lk, Hq, Hkv, D, BS, window, dtype = case
    q, kc, vc, cuq, cuk, table = _case(22, lq, lk, Hq, Hkv, D, BS, dtype)
    kcont, vcont = _contiguous(kc, cuk, table), _contiguous(vc, cuk, table)
    print(f"prefill contiguous lq={lq} lk={lk} D={D} w={window}", flush=True)
    paged = _gpu(device, q, kc, vc, cuq, cuk, table, 0.1, window, dtype)
    cont = _gpu(device, q, kcont, vcont, cuq, cuk, table, 0.1, window, dtype, paged=False)
    assert torch.equal(paged, cont)
    want = oracle.prefill_attention(q, kcont, vcont, cuq, cuk, 0.1, None, window, dtype)
    assert_attn_close(to_f32(cont), want)


def test_prefill_placement_invariance(device):
    """Moving blocks to other physical ids (same logical content) changes nothing, bit for bit."""
    import torch

    lq, lk = [100, 60], [700, 60]
    q, kc, vc, cuq, cuk, table = _case(23, lq, lk, 32, 8, 128, 16, "bf16", spare=30)
    NB = kc.shape[0]
    perm = np.random.default_rng(5).permutation(NB).astype(np.int32)
    kc2 = np.empty_like(kc)
    vc2 = np.empty_like(vc)
    kc2[perm] = kc
    vc2[perm] = vc
    table2 = perm[table]
    a = _gpu(device, q, kc, vc, cuq, cuk, table, 0.08, -1, "bf16")
    b = _gpu(device, q, kc2, vc2, cuq, cuk, table2, 0.08, -1, "bf16")
    assert torch.equal(a, b)


def test_prefill_long_prompt_rows_vs_decode_oracle(device):
    """Two 4096-token prompts behind a 1000-token prefix (Qwen3-8B heads): sampled rows
    checked against the decode oracle over each row's causal prefix."""
    lq, lk = [4096, 2500], [5096, 2500]
    q, kc, vc, cuq, cuk, table = _case(24, lq, lk, 32, 8, 128, 256, "bf16")
    scale = 1 / math.sqrt(128)
    print("prefill long prompt 4096+2500", flush=True)
    got = to_f32(_gpu(device, q, kc, vc, cuq, cuk, table, scale, -1, "bf16"))
    rng = np.random.default_rng(0)
    for b in range(2):
        for i in np.concatenate([[0, lq[b] - 1], rng.integers(0, lq[b], 6)]):
            L = int(i) + lk[b] - lq[b] + 1
            t = int(cuq[b]) + int(i)
            want = oracle.paged_decode_attention(q[t][None], kc, vc, np.array([0, L], np.uint32),
                                                 table[b][None], scale, -1, "bf16")
            assert_attn_close(got[t][None], want)


def test_prefill_rejects_bad_arguments(device):
    import torch
    import oxide_paged_kv as ox

    q = torch.zeros((4, 8, 96), dtype=torch.bfloat16, device=device)  # head_dim 96: not built
    cu = torch.tensor([0, 4], dtype=torch.int32, device=device)
    with pytest.raises(ox.OxideError):
        ox.prefill_attn(q, q, q, cu, cu, 4, 4, 1.0)
    q = torch.zeros((4, 8, 128), dtype=torch.float32, device=device)  # f32: not supported
    with pytest.raises(ox.OxideError):
        ox.prefill_attn(q, q, q, cu, cu, 4, 4, 1.0)


@pytest.mark.parametrize("window", [-1, 300])
def test_prefill_last_rows_equal_decode(device, window):
    """Cross-kernel invariant: the last query row of every prompt sees exactly the keys a
    decode step over the same cache sees, so the two kernels agree (within the
    attention tolerance: different accumulation orders)."""
    import torch
    import oxide_paged_kv as ox
    from helpers import assert_attn_close

    lq, lk = [200, 77, 1, 513], [1200, 77, 40, 513]
    q, kc, vc, cuq, cuk, table = _case(25, lq, lk, 32, 8, 128, 256, "bf16")
    pre = to_f32(_gpu(device, q, kc, vc, cuq, cuk, table, 0.09, window, "bf16"))
    last = np.array([int(cuq[b + 1]) - 1 for b in range(len(lq))])
    dec = ox.decode_attn(to_torch(q[last], "bf16", device), to_torch(kc, "bf16", device),
                         to_torch(vc, "bf16", device), torch.from_numpy(cuk.view(np.int32)).to(device),
                         torch.from_numpy(table).to(device), max(lk), 0.09, None if window < 0 else window)
    torch.cuda.synchronize()
    assert_attn_close(pre[last], to_f32(dec))
