"""GPU parity of the fused attention prologue (q/k RMSNorm + RoPE + KV append) against
the oracle.

Bar: v rows in the cache are bit-exact (a copy).  q and k follow the reference's
rounding steps; with the norm the only freedom left is the order of the fp32 sum of
squares (a tree sum on the GPU, an fp64 sum in the oracle), which may move a normed
element by one unit in the last place of the 16-bit format before the rotation: the
rotated outputs may then differ by that unit carried through the rotation (bounded by
the pair's magnitude, see _assert_rotated), and at most 2 % of them may differ at all.
Inputs whose sums of squares are exact in any order must agree bit for bit.  Without the norm (the qkv-bias models) there is no reduction and
the result must be bit-exact.
"""
import numpy as np
import pytest

import oracle
from helpers import normal_bits, to_bits, to_torch

pytestmark = pytest.mark.gpu


def _ordered(bits):
    """16-bit float patterns -> integers whose order and spacing follow the values (1 = 1 ulp)."""
    b = bits.astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def _assert_ulp(got, want, max_frac):
    d = np.abs(_ordered(got) - _ordered(want))
    assert d.max() <= 1, f"max ulp difference {d.max()}"
    frac = float((d > 0).mean())
    assert frac <= max_frac, f"{frac:.4f} of elements differ"
    return frac


def _ulp16(x, dtype):
    """Spacing of the 16-bit format at |x| (its subnormal spacing below the normal range)."""
    mant, emin = (7, -126) if dtype == "bf16" else (10, -14)
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** emin)))
    return np.exp2(e - mant)


def _assert_rotated(got, want, dtype, D, max_frac):
    """Rotated q / k rows.  The sum-of-squares order may move a normed element by one
    ulp before the rotation, which carries it into y1 = x1 c - x2 s (or y2) as up to
    one ulp of the pair's magnitude hypot(y1, y2) (the rotation preserves it) per
    operand -- many ulps of y itself where the two products cancel.  Bar: |got - want|
    <= 2 ulp(hypot) + ulp(want) everywhere, and at most max_frac of the elements differ."""
    g = oracle.bits_to_f32(got.reshape(-1, D), dtype).astype(np.float64)
    w = oracle.bits_to_f32(want.reshape(-1, D), dtype).astype(np.float64)
    partner = np.concatenate([w[:, D // 2:], w[:, :D // 2]], axis=1)
    bound = 2 * _ulp16(np.hypot(w, partner), dtype) + _ulp16(w, dtype)
    err = np.abs(g - w)
    assert np.all(err <= bound), f"max error / bound {float((err / bound).max()):.2f}"
    frac = float((got != want).mean())
    assert frac <= max_frac, f"{frac:.4f} of elements differ"


def _case(seed, T, Hq, Hkv, D, dtype, weights, pad=0):
    rng = np.random.default_rng(seed)
    row = (Hq + 2 * Hkv) * D
    qkv = normal_bits(rng, (T, row + pad), dtype, 2.0)
    if weights:
        w = oracle.half_to_float(normal_bits(rng, (2, D), dtype, 0.1), dtype) + 1.0
        wq, wk = oracle.float_to_half(w[0], dtype), oracle.float_to_half(w[1], dtype)
    else:
        wq = wk = None
    pos = rng.integers(0, 8192, T).astype(np.int32)
    pos[0] = 0
    return qkv, wq, wk, pos


CASES = [
    # (T, Hq, Hkv, D, dtype, weights, pad)
    (37, 32, 8, 128, "bf16", True, 0),    # Qwen3-8B heads
    (64, 64, 8, 128, "bf16", True, 0),    # Qwen3-32B heads
    (20, 16, 8, 128, "f16", True, 0),     # f16
    (11, 8, 4, 64, "bf16", True, 0),      # D = 64
    (9, 16, 8, 128, "bf16", False, 0),    # no q/k norm: rope only, bit-exact
    (13, 4, 2, 64, "f16", False, 3),      # row stride not a multiple of 8: element copy of v
    # Beyond the resident grid (16 workgroups per CU x 256 CUs x 32 or 64 tasks): each
    # lane walks several tasks with the next one prefetched; T leaves a ragged last round.
    (4099, 32, 8, 128, "bf16", True, 0),
    (12007, 16, 4, 64, "f16", True, 3),   # the same through the per-element kernel
]


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_prologue_vs_oracle(device, case):
    import torch
    import oxide_paged_kv as ox

    T, Hq, Hkv, D, dtype, weights, pad = case
    print(f"prologue case T={T} Hq={Hq} Hkv={Hkv} D={D} {dtype} norm={weights} pad={pad}", flush=True)
    qkv, wq, wk, pos = _case(7, T, Hq, Hkv, D, dtype, weights, pad)
    cs = oracle.rope_cos_sin_cache(8192, D, 1_000_000.0)
    BS = 16
    NB = max(6, -(-3 * T // (2 * BS)))  # room for every token and some free slots
    rng = np.random.default_rng(1)
    slots = rng.permutation(NB * BS)[:T].astype(np.int64)
    slots[1::5] = -1
    kc = normal_bits(rng, (NB, BS, Hkv, D), dtype)
    vc = normal_bits(rng, (NB, BS, Hkv, D), dtype)
    kc_want, vc_want = kc.copy(), vc.copy()
    row = (Hq + 2 * Hkv) * D
    q_want, k_want = oracle.qk_norm_rope_and_cache(qkv[:, :row] if pad == 0 else np.ascontiguousarray(qkv[:, :row]),
                                                   Hq, Hkv, D, wq, wk, 1e-6, cs, pos, kc_want, vc_want,
                                                   slots, dtype)
    t = lambda a: to_torch(a, dtype, device)  # noqa: E731
    kc_g, vc_g = t(kc), t(vc)
    q, k = ox.qk_norm_rope_and_cache(t(qkv)[:, :row] if pad else t(qkv), Hq, Hkv,
                                     t(wq) if weights else None, t(wk) if weights else None, 1e-6,
                                     torch.from_numpy(cs).to(device), torch.from_numpy(pos).to(device),
                                     kc_g, vc_g, torch.from_numpy(slots).to(device), return_k=True)
    torch.cuda.synchronize()
    assert np.array_equal(to_bits(vc_g), vc_want)
    if weights:
        _assert_rotated(to_bits(q), q_want, dtype, D, 0.02)
        _assert_rotated(to_bits(k), k_want, dtype, D, 0.02)
        _assert_rotated(to_bits(kc_g), kc_want, dtype, D, 0.02)
    else:
        assert np.array_equal(to_bits(q), q_want)
        assert np.array_equal(to_bits(k), k_want)
        assert np.array_equal(to_bits(kc_g), kc_want)
    # Cache rows of skipped tokens and unused slots are untouched.
    used = set(int(s) for s in slots if s >= 0)
    free = [i for i in range(NB * BS) if i not in used]
    assert np.array_equal(to_bits(kc_g).reshape(NB * BS, -1)[free], kc.reshape(NB * BS, -1)[free])


def test_prologue_then_decode_attention_matches_oracle_chain(device):
    """Decode step in the engine's order: prologue (norm + rope + append of the new token)
    then paged decode attention; checked against the oracle running the same chain."""
    import math

    import torch
    import oxide_paged_kv as ox
    from helpers import assert_attn_close, to_f32

    B, Hq, Hkv, D, BS = 6, 32, 8, 128, 256
    rng = np.random.default_rng(3)
    lens = np.array([1, 300, 257, 1024, 2, 700])
    nblk = (lens + BS - 1) // BS
    NB = int(nblk.sum()) + 1
    perm = rng.permutation(NB).astype(np.int32)
    table = np.zeros((B, nblk.max()), np.int32)
    pos0 = 0
    for b in range(B):
        table[b, :nblk[b]] = perm[pos0:pos0 + nblk[b]]
        pos0 += nblk[b]
    cu = np.zeros(B + 1, np.uint32)
    cu[1:] = np.cumsum(lens)
    slots = np.array([table[b, (L - 1) // BS] * BS + (L - 1) % BS for b, L in enumerate(lens)], np.int64)
    positions = (lens - 1).astype(np.int32)
    qkv, wq, wk, _ = _case(9, B, Hq, Hkv, D, "bf16", True)
    kc = normal_bits(rng, (NB, BS, Hkv, D), "bf16")
    vc = normal_bits(rng, (NB, BS, Hkv, D), "bf16")
    cs = oracle.rope_cos_sin_cache(4096, D, 1_000_000.0)
    scale = 1 / math.sqrt(D)

    kc_o, vc_o = kc.copy(), vc.copy()
    q_o, _ = oracle.qk_norm_rope_and_cache(qkv, Hq, Hkv, D, wq, wk, 1e-6, cs, positions, kc_o, vc_o, slots)
    want = oracle.paged_decode_attention(q_o, kc_o, vc_o, cu, table, scale)

    t = lambda a: to_torch(a, "bf16", device)  # noqa: E731
    kc_g, vc_g = t(kc), t(vc)
    sm = torch.from_numpy(slots).to(device)
    q = ox.qk_norm_rope_and_cache(t(qkv), Hq, Hkv, t(wq), t(wk), 1e-6, torch.from_numpy(cs).to(device),
                                  torch.from_numpy(positions).to(device), kc_g, vc_g, sm)
    out = ox.decode_attn(q, kc_g, vc_g, torch.from_numpy(cu.view(np.int32)).to(device),
                         torch.from_numpy(table).to(device), int(lens.max()), scale)
    torch.cuda.synchronize()
    assert_attn_close(to_f32(out), want)


def test_rope_cache_builder_matches_oracle(device):
    import oxide_paged_kv as ox

    got = ox.rope_cos_sin_cache(4096, 128, 1_000_000.0).numpy()
    want = oracle.rope_cos_sin_cache(4096, 128, 1_000_000.0)
    assert np.array_equal(got, want)


def test_prologue_without_append(device):
    """slot_mapping None: q (and k) are produced, nothing is written to any cache."""
    import torch
    import oxide_paged_kv as ox

    qkv, wq, wk, pos = _case(8, 5, 8, 4, 128, "bf16", True)
    cs = oracle.rope_cos_sin_cache(8192, 128, 1_000_000.0)
    q_want, k_want = oracle.qk_norm_rope_and_cache(qkv, 8, 4, 128, wq, wk, 1e-6, cs, pos)
    t = lambda a: to_torch(a, "bf16", device)  # noqa: E731
    q, k = ox.qk_norm_rope_and_cache(t(qkv), 8, 4, t(wq), t(wk), 1e-6, torch.from_numpy(cs).to(device),
                                     torch.from_numpy(pos).to(device), return_k=True)
    torch.cuda.synchronize()
    _assert_rotated(to_bits(q), q_want, "bf16", 128, 0.02)
    _assert_rotated(to_bits(k), k_want, "bf16", 128, 0.02)


def _exact_sum_case(seed, T, Hq, Hkv, D, dtype, tiny_heads=()):
    """qkv rows whose sums of squares are exact in any order: elements k / 8 with
    |k| <= 16 (squares are multiples of 2^-6, a head's sum stays below 2^11), so
    GPU and oracle see the same mean and the whole chain must agree bit for bit.
    Heads listed in tiny_heads hold k * 2^-70 instead: below the fast divide's
    domain, so they take the general divide (eps dominates their mean)."""
    rng = np.random.default_rng(seed)
    H = Hq + 2 * Hkv
    x = (rng.integers(-16, 17, (T, H, D)) / 8.0).astype(np.float32)
    for h in tiny_heads:
        x[:, h, :] = rng.integers(-16, 17, (T, D)).astype(np.float32) * np.float32(2.0 ** -70)
    x[0, 0, :3] = 0.0
    x[0, 0, 3] = -0.0
    qkv = oracle.float_to_half(x.reshape(T, H * D), dtype)
    w = oracle.float_to_half(1.0 + rng.integers(-8, 9, (2, D)) / 64.0, dtype)
    pos = rng.integers(0, 8192, T).astype(np.int32)
    return qkv, w[0], w[1], pos


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("D", [128, 64])
def test_prologue_bit_exact_when_sums_are_exact(device, dtype, D):
    """Pins the per-element arithmetic (the divide by the rms, both roundings, the
    weight, the rotation) bit for bit: the only freedom, the order of the sum of
    squares, is removed by inputs whose sums are exact.  Heads 1 (a q head) and
    Hq + 1 (a k head) take the general-divide path."""
    import torch
    import oxide_paged_kv as ox

    T, Hq, Hkv = 33, 16, 4
    print(f"prologue exact-sum D={D} {dtype}", flush=True)
    tiny = (1, Hq + 1) if dtype == "bf16" else ()
    qkv, wq, wk, pos = _exact_sum_case(11, T, Hq, Hkv, D, dtype, tiny_heads=tiny)
    cs = oracle.rope_cos_sin_cache(8192, D, 1_000_000.0)
    q_want, k_want = oracle.qk_norm_rope_and_cache(qkv, Hq, Hkv, D, wq, wk, 1e-6, cs, pos, dtype=dtype)
    t = lambda a: to_torch(a, dtype, device)  # noqa: E731
    q, k = ox.qk_norm_rope_and_cache(t(qkv), Hq, Hkv, t(wq), t(wk), 1e-6, torch.from_numpy(cs).to(device),
                                     torch.from_numpy(pos).to(device), return_k=True)
    torch.cuda.synchronize()
    got_q, got_k = to_bits(q), to_bits(k)
    assert np.array_equal(got_q, q_want), f"{int((got_q != q_want).sum())} q elements differ"
    assert np.array_equal(got_k, k_want), f"{int((got_k != k_want).sum())} k elements differ"
    if tiny:
        assert got_q.reshape(T, Hq, D)[:, 1].any()  # the tiny heads did not flush to zero


def test_prologue_nan_propagates(device):
    """A NaN input element makes NaN outputs where the oracle has them (payload bits
    after fp32 arithmetic are the hardware's own, so NaN-ness is compared), and the
    rest of the head and of the batch is unaffected."""
    import torch
    import oxide_paged_kv as ox

    T, Hq, Hkv, D = 4, 8, 2, 128
    qkv, wq, wk, pos = _case(12, T, Hq, Hkv, D, "bf16", True)
    qkv[1, 5 * D + 7] = 0x7FC1           # q head 5 of token 1 (normed: the whole head turns NaN)
    qkv[2, (Hq + 1) * D + 3] = 0xFF80    # -inf in k head 1 of token 2
    cs = oracle.rope_cos_sin_cache(8192, D, 1_000_000.0)
    q_want, k_want = oracle.qk_norm_rope_and_cache(qkv, Hq, Hkv, D, wq, wk, 1e-6, cs, pos)
    t = lambda a: to_torch(a, "bf16", device)  # noqa: E731
    q, k = ox.qk_norm_rope_and_cache(t(qkv), Hq, Hkv, t(wq), t(wk), 1e-6, torch.from_numpy(cs).to(device),
                                     torch.from_numpy(pos).to(device), return_k=True)
    torch.cuda.synchronize()
    for got, want in ((to_bits(q), q_want), (to_bits(k), k_want)):
        gf = oracle.half_to_float(got, "bf16")
        wf = oracle.half_to_float(want, "bf16")
        assert np.array_equal(np.isnan(gf), np.isnan(wf))
        fin = ~np.isnan(wf)
        _assert_ulp(got[fin], want[fin], 0.02)
    assert np.isnan(oracle.half_to_float(q_want, "bf16")).any()


def test_prologue_preallocated_outputs(device):
    """q_out / k_out: results land in the caller's buffers, identical to fresh ones;
    wrong shapes are refused."""
    import torch
    import oxide_paged_kv as ox

    qkv, wq, wk, pos = _case(13, 7, 8, 2, 128, "bf16", True)
    cs = torch.from_numpy(oracle.rope_cos_sin_cache(8192, 128, 1_000_000.0)).to(device)
    t = lambda a: to_torch(a, "bf16", device)  # noqa: E731
    args = (t(qkv), 8, 2, t(wq), t(wk), 1e-6, cs, torch.from_numpy(pos).to(device))
    q, k = ox.qk_norm_rope_and_cache(*args, return_k=True)
    qo = torch.full((7, 8, 128), 7.0, dtype=torch.bfloat16, device=device)
    ko = torch.full((7, 2, 128), 7.0, dtype=torch.bfloat16, device=device)
    q2, k2 = ox.qk_norm_rope_and_cache(*args, q_out=qo, k_out=ko)
    torch.cuda.synchronize()
    assert q2 is qo and k2 is ko
    assert torch.equal(qo, q) and torch.equal(ko, k)
    with pytest.raises(ox.OxideError):
        ox.qk_norm_rope_and_cache(*args, q_out=torch.empty((7, 8, 64), dtype=torch.bfloat16, device=device))
