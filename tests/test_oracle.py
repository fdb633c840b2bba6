"""Pins the C oracle (CPU only) against the reference's golden vectors, independent
library routines (numpy, torch, python-xxhash) and closed forms.  Each test names
what a plausible oracle mistake would break."""
import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle
from helpers import normal_bits

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


# ------------------------------------------------------------------ formats
def test_bf16_rounding_matches_torch():
    import torch

    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-30, 30, 20000).astype(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 3.3895e38, 1e-40],
                 dtype=np.float32)])
    want = torch.from_numpy(x).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.float_to_half(x, "bf16"), want)
    assert np.array_equal(oracle.f32_to_bf16_bits(x[np.isfinite(x)]), want[np.isfinite(x)])
    back = oracle.half_to_float(want, "bf16")
    assert np.array_equal(back.view(np.uint32), (want.astype(np.uint32) << 16))


def test_f16_rounding_matches_numpy():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(2.0) ** rng.integers(-30, 18, 20000).astype(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65519.99, 65520, 2**-24, 2**-25, 3 * 2**-26,
                  2**-14 - 2**-25, 1e-8], dtype=np.float32)])
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.float_to_half(x, "f16"), want)
    allbits = np.arange(65536, dtype=np.uint16)
    ok = ~np.isnan(allbits.view(np.float16))
    got = oracle.half_to_float(allbits, "f16")
    assert np.array_equal(got[ok], allbits[ok].view(np.float16).astype(np.float32))


# --------------------------------------------------------------- host logic
@pytest.mark.parametrize("case", GOLDEN["slot_mapping"], ids=lambda c: c["cite"].split()[-1])
def test_slot_mapping_reference_known_answers(case):
    got = oracle.compute_slot_mapping(case["block_table"], case["block_size"], case["token_offset"],
                                      case["num_tokens"])
    assert got.tolist() == case["expected"]


def test_slot_mapping_full_range():
    c = GOLDEN["slot_mapping_full_range"]
    got = oracle.compute_slot_mapping(c["block_table"], c["block_size"], 0, c["num_tokens"])
    bt = c["block_table"]
    assert got.tolist() == [bt[i // 256] * 256 + i % 256 for i in range(c["num_tokens"])]


@pytest.mark.parametrize("case", GOLDEN["decode_metadata"], ids=lambda c: c["cite"].split()[-1])
def test_decode_metadata_reference_known_answers(case):
    cu_q, cu_k, mx = oracle.build_decode_metadata(case["context_lens"])
    assert cu_q.tolist() == case["cu_seqlens_q"]
    assert cu_k.tolist() == case["cu_seqlens_k"]
    assert mx == case["max_seqlen_k"]


def test_pad_block_table():
    rows = [[7, 3], [], [1, 2, 9, 4], [5]]
    got = oracle.pad_block_table(rows)
    assert got.tolist() == [[7, 3, 0, 0], [0, 0, 0, 0], [1, 2, 9, 4], [5, 0, 0, 0]]


# ------------------------------------------------------------ cache copies
def test_reshape_and_cache_reference_known_answer():
    ka = GOLDEN["reshape_and_cache_known_answer"]
    T, H, D, NB, BS = ka["num_tokens"], ka["num_kv_heads"], ka["head_dim"], ka["num_blocks"], ka["block_size"]
    key = oracle.f32_to_bf16_bits(np.arange(T * H * D, dtype=np.float32)).reshape(T, H, D)
    val = oracle.f32_to_bf16_bits(1000 + np.arange(T * H * D, dtype=np.float32)).reshape(T, H, D)
    kc = np.zeros((NB, BS, H, D), np.uint16)
    vc = np.zeros_like(kc)
    oracle.reshape_and_cache(key, val, kc, vc, np.array(ka["slot_mapping"], np.int64))
    assert np.array_equal(kc[0, 0], key[0]) and np.array_equal(kc[1, 0], key[1])
    assert np.array_equal(vc[2, 0], val[2])
    assert np.count_nonzero(kc) == np.count_nonzero(key)


def test_reshape_and_cache_matches_fancy_index_and_skips_minus_one():
    rng = np.random.default_rng(3)
    NB, BS, H, D, T = 5, 16, 2, 8, 40
    kc = rng.integers(0, 65535, (NB, BS, H, D)).astype(np.uint16)
    vc = rng.integers(0, 65535, (NB, BS, H, D)).astype(np.uint16)
    key = rng.integers(0, 65535, (T, H, D)).astype(np.uint16)
    val = rng.integers(0, 65535, (T, H, D)).astype(np.uint16)
    slots = rng.choice(NB * BS, T, replace=False).astype(np.int64)
    slots[3::5] = -1
    ek, ev = kc.copy().reshape(-1, H, D), vc.copy().reshape(-1, H, D)
    keep = slots >= 0
    ek[slots[keep]] = key[keep]
    ev[slots[keep]] = val[keep]
    oracle.reshape_and_cache(key, val, kc, vc, slots)
    assert np.array_equal(kc.reshape(-1, H, D), ek) and np.array_equal(vc.reshape(-1, H, D), ev)


def test_copy_and_gather_match_fancy_index():
    rng = np.random.default_rng(4)
    kc = rng.integers(0, 2**32, (8, 4, 3, 5), dtype=np.uint64).astype(np.uint32)
    vc = rng.integers(0, 2**32, (8, 4, 3, 5), dtype=np.uint64).astype(np.uint32)
    mapping = np.array([[0, 5], [2, 6], [3, 3]], np.int64)
    ek, ev = kc.copy(), vc.copy()
    ek[mapping[:, 1]] = kc[mapping[:, 0]]
    ev[mapping[:, 1]] = vc[mapping[:, 0]]
    oracle.copy_blocks(kc, vc, mapping)
    assert np.array_equal(kc, ek) and np.array_equal(vc, ev)
    ids = np.array([7, 0, 6], np.int32)
    gk, gv = oracle.gather_blocks(kc, vc, ids)
    assert np.array_equal(gk, kc[ids]) and np.array_equal(gv, vc[ids])


# --------------------------------------------------------------- attention
def _rand_case(seed, B, Hq, Hkv, D, BS, NB, lens, dtype="bf16"):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens)
    nblk = (lens + BS - 1) // BS
    perm = rng.permutation(NB).astype(np.int32)
    table = np.zeros((B, max(int(nblk.max()), 1)), np.int32)
    pos = 0
    for b in range(B):
        table[b, :nblk[b]] = perm[pos:pos + nblk[b]]
        pos += nblk[b]
    cu = np.zeros(B + 1, np.uint32)
    cu[1:] = np.cumsum(lens)
    return (normal_bits(rng, (B, Hq, D), dtype), normal_bits(rng, (NB, BS, Hkv, D), dtype),
            normal_bits(rng, (NB, BS, Hkv, D), dtype), cu, table)


def _numpy_f64_attention(q, kc, vc, cu, table, scale, window, dtype):
    """Independent textbook routine: gather contiguous K/V with numpy fancy indexing,
    then softmax(scale q K^T) V in float64."""
    B, Hq, D = q.shape
    NB, BS, Hkv, _ = kc.shape
    G = Hq // Hkv
    qf = oracle.bits_to_f32(q, dtype).astype(np.float64)
    kf = oracle.bits_to_f32(kc, dtype).astype(np.float64)
    vf = oracle.bits_to_f32(vc, dtype).astype(np.float64)
    out = np.zeros((B, Hq, D))
    for b in range(B):
        L = int(cu[b + 1] - cu[b])
        if L == 0:
            continue
        j = np.arange(L)
        rows = table[b, j // BS].astype(np.int64) * BS + j % BS
        K = kf.reshape(-1, Hkv, D)[rows]  # [L, Hkv, D]
        V = vf.reshape(-1, Hkv, D)[rows]
        lo = 0 if window < 0 else max(0, L - 1 - window)
        for h in range(Hq):
            s = K[lo:, h // G] @ qf[b, h] * scale
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ V[lo:, h // G]
    return out


@pytest.mark.parametrize("G,D,BS,window,dtype", [(2, 128, 256, -1, "bf16"), (4, 128, 16, 37, "bf16"),
                                                 (1, 64, 32, -1, "f16"), (8, 64, 256, 300, "f16")])
def test_attention_matches_numpy_f64(G, D, BS, window, dtype):
    Hkv = 2
    q, kc, vc, cu, table = _rand_case(5, 3, G * Hkv, Hkv, D, BS, 80, [700, 1, 0], dtype)
    scale = 1 / math.sqrt(D)
    want = _numpy_f64_attention(q, kc, vc, cu, table, scale, window, dtype)
    got32 = oracle.paged_decode_attention(q, kc, vc, cu, table, scale, window, dtype)
    got64 = oracle.paged_decode_attention(q, kc, vc, cu, table, scale, window, dtype, use_f64=True)
    np.testing.assert_allclose(got64, want, atol=1e-7, rtol=1e-6)  # fp32 output rounding
    np.testing.assert_allclose(got32, want, atol=2e-5, rtol=1e-4)
    # Wrong kv-head mapping (h % Hkv instead of h // G) must be caught: heads differ.
    assert not np.allclose(want[0, 0], want[0, -1])


def test_attention_closed_forms():
    q, kc, vc, cu, table = _rand_case(6, 2, 8, 2, 64, 16, 40, [100, 1])
    scale = 0.125
    # L = 1: output is v_0 exactly.
    out = oracle.paged_decode_attention(q, kc, vc, cu, table, scale, -1, "bf16")
    v0 = oracle.bits_to_f32(vc[table[1, 0], 0], "bf16")
    assert np.array_equal(out[1], np.repeat(v0, 4, axis=0))
    # q = 0: uniform weights -> mean of V over the window.
    qz = np.zeros_like(q)
    out = oracle.paged_decode_attention(qz, kc, vc, cu, table, scale, 9, "bf16")
    j = np.arange(90, 100)
    rows = table[0, j // 16].astype(np.int64) * 16 + j % 16
    Vw = oracle.bits_to_f32(vc.reshape(-1, 2, 64)[rows], "bf16")
    np.testing.assert_allclose(out[0, :4], np.repeat(Vw[:, 0].mean(0)[None], 4, 0), atol=1e-6)
    np.testing.assert_allclose(out[0, 4:], np.repeat(Vw[:, 1].mean(0)[None], 4, 0), atol=1e-6)
    # A huge score on one key: output is that key's V row.
    kc2 = np.zeros_like(kc)
    blk, off = table[0, 3], 5  # key 53
    kc2[blk, off, 0] = oracle.f32_to_bf16_bits(np.full(64, 8.0, np.float32))
    q1 = oracle.f32_to_bf16_bits(np.full(q.shape, 8.0, np.float32))
    out = oracle.paged_decode_attention(q1, kc2, vc, cu, table, 1.0, -1, "bf16")
    np.testing.assert_allclose(out[0, 0], oracle.bits_to_f32(vc[blk, off, 0], "bf16"), atol=1e-6)


def test_attention_window_edge_counts_w_plus_one_keys():
    """window_left = w admits keys [L-1-w, L-1]: w + 1 keys (FA2 convention)."""
    q, kc, vc, cu, table = _rand_case(7, 1, 2, 1, 64, 16, 10, [50])
    qz = np.zeros_like(q)
    out = oracle.paged_decode_attention(qz, kc, vc, cu, table, 1.0, 2, "bf16")
    j = np.array([47, 48, 49])
    rows = table[0, j // 16].astype(np.int64) * 16 + j % 16
    want = oracle.bits_to_f32(vc.reshape(-1, 1, 64)[rows, 0], "bf16").mean(0)
    np.testing.assert_allclose(out[0, 0], want, atol=1e-6)


# ------------------------------------------------------------------ prefill
def _prefill_case(seed, lq, lk, Hq, Hkv, D, BS, NB, dtype="bf16"):
    rng = np.random.default_rng(seed)
    _, kc, vc, cuk, table = _rand_case(seed, len(lk), Hq, Hkv, D, BS, NB, lk, dtype)
    cuq = np.zeros(len(lq) + 1, np.uint32)
    cuq[1:] = np.cumsum(lq)
    q = normal_bits(rng, (int(cuq[-1]), Hq, D), dtype)
    return q, kc, vc, cuq, cuk, table


def _numpy_f64_prefill(q, kc, vc, cuq, cuk, table, scale, window, dtype):
    """Independent dense routine: gather K/V, full [Lq, Lk] score matrix, boolean
    mask from the FlashAttention 2 bottom-right rule, masked softmax in float64."""
    Tq, Hq, D = q.shape
    NB, BS, Hkv, _ = kc.shape
    G = Hq // Hkv
    qf = oracle.bits_to_f32(q, dtype).astype(np.float64)
    kf = oracle.bits_to_f32(kc, dtype).astype(np.float64).reshape(-1, Hkv, D)
    vf = oracle.bits_to_f32(vc, dtype).astype(np.float64).reshape(-1, Hkv, D)
    out = np.zeros((Tq, Hq, D))
    for b in range(len(cuq) - 1):
        q0, Lq = int(cuq[b]), int(cuq[b + 1] - cuq[b])
        Lk = int(cuk[b + 1] - cuk[b])
        if Lq == 0 or Lk == 0:
            continue
        j = np.arange(Lk)
        rows = table[b, j // BS].astype(np.int64) * BS + j % BS
        ii, jj = np.meshgrid(np.arange(Lq), j, indexing="ij")
        mask = jj <= ii + Lk - Lq
        if window >= 0:
            mask &= jj >= ii + Lk - Lq - window
        for h in range(Hq):
            s = qf[q0:q0 + Lq, h] @ kf[rows, h // G].T * scale
            s = np.where(mask, s, -np.inf)
            m = s.max(axis=1, keepdims=True)
            m = np.where(np.isfinite(m), m, 0.0)
            p = np.exp(s - m)
            den = p.sum(axis=1, keepdims=True)
            o = (p @ vf[rows, h // G]) / np.where(den > 0, den, 1.0)
            out[q0:q0 + Lq, h] = o
    return out


@pytest.mark.parametrize("G,D,BS,window,dtype", [(4, 128, 256, -1, "bf16"), (2, 64, 16, 23, "bf16"),
                                                 (1, 128, 32, -1, "f16"), (8, 64, 64, 100, "f16")])
def test_prefill_matches_numpy_f64(G, D, BS, window, dtype):
    Hkv = 2
    # prompt without prefix, prompt after a cached prefix, Lk < Lq, empty query list
    lq, lk = [37, 20, 9, 0], [37, 150, 4, 30]
    q, kc, vc, cuq, cuk, table = _prefill_case(11, lq, lk, G * Hkv, Hkv, D, BS, 40, dtype)
    scale = 1 / math.sqrt(D)
    want = _numpy_f64_prefill(q, kc, vc, cuq, cuk, table, scale, window, dtype)
    got64 = oracle.prefill_attention(q, kc, vc, cuq, cuk, scale, table, window, dtype, use_f64=True)
    got32 = oracle.prefill_attention(q, kc, vc, cuq, cuk, scale, table, window, dtype)
    np.testing.assert_allclose(got64, want, atol=1e-7, rtol=1e-6)
    np.testing.assert_allclose(got32, want, atol=2e-5, rtol=1e-4)
    # Lq = 9 with Lk = 4: queries 0..4 see no key (hi < 0) and are zero.
    assert np.all(got64[57:62] == 0) and np.any(got64[62] != 0)


def test_prefill_rows_equal_decode_over_their_prefix():
    """Query i of a sequence is a decode call whose context is keys [0, i + Lk - Lq]."""
    lq, lk = [12, 7], [12, 300]
    q, kc, vc, cuq, cuk, table = _prefill_case(12, lq, lk, 8, 2, 64, 16, 40)
    for window in (-1, 5):
        got = oracle.prefill_attention(q, kc, vc, cuq, cuk, 0.2, table, window)
        for b in range(2):
            for i in range(lq[b]):
                L = i + lk[b] - lq[b] + 1
                t = int(cuq[b]) + i
                dec = oracle.paged_decode_attention(q[t][None], kc, vc, np.array([0, L], np.uint32),
                                                    table[b][None], 0.2, window)
                assert np.array_equal(got[t], dec[0]), (b, i, window)


def test_prefill_fa2_bottom_right_mask_hand_case():
    """Lq = 2, Lk = 5, q = 0 (uniform weights): query 0 averages keys 0..3 and
    query 1 keys 0..4; with window_left = 1, keys 2..3 and 3..4."""
    q, kc, vc, cuq, cuk, table = _prefill_case(13, [2], [5], 1, 1, 64, 16, 4)
    qz = np.zeros_like(q)
    V = oracle.bits_to_f32(vc[table[0, 0], :5, 0], "bf16").astype(np.float64)
    out = oracle.prefill_attention(qz, kc, vc, cuq, cuk, 1.0, table, -1, use_f64=True)
    np.testing.assert_allclose(out[0, 0], V[:4].mean(0), atol=1e-6)
    np.testing.assert_allclose(out[1, 0], V[:5].mean(0), atol=1e-6)
    out = oracle.prefill_attention(qz, kc, vc, cuq, cuk, 1.0, table, 1, use_f64=True)
    np.testing.assert_allclose(out[0, 0], V[2:4].mean(0), atol=1e-6)
    np.testing.assert_allclose(out[1, 0], V[3:5].mean(0), atol=1e-6)


def test_prefill_contiguous_equals_paged():
    lq, lk = [20, 33], [50, 33]
    q, kc, vc, cuq, cuk, table = _prefill_case(14, lq, lk, 4, 2, 64, 16, 20)
    rows = np.concatenate([table[b, np.arange(lk[b]) // 16].astype(np.int64) * 16 + np.arange(lk[b]) % 16
                           for b in range(2)])
    kcont = kc.reshape(-1, 2, 64)[rows]
    vcont = vc.reshape(-1, 2, 64)[rows]
    paged = oracle.prefill_attention(q, kc, vc, cuq, cuk, 0.3, table, 7)
    cont = oracle.prefill_attention(q, kcont, vcont, cuq, cuk, 0.3, None, 7)
    assert np.array_equal(paged, cont)


# ------------------------------------------------------------------- xxh64
def test_xxh64_matches_python_xxhash():
    import xxhash

    rng = np.random.default_rng(8)
    assert oracle.xxh64(b"", 0) == 0xEF46DB3751D8E999  # spec's empty-input digest
    for n in [0, 1, 3, 4, 7, 8, 31, 32, 33, 63, 64, 100, 1027]:
        data = rng.integers(0, 256, n).astype(np.uint8).tobytes()
        for seed in (0, 1, 2**63 + 5):
            assert oracle.xxh64(data, seed) == xxhash.xxh64_intdigest(data, seed=seed)


# ------------------------------------------------------ norm + rope prologue
def test_rope_cos_sin_cache_formula_and_reference_tests():
    """layers/rope.rs:50-83: f_i = 1 / base^(2i/R) (fp32), row t = [cos(t f), sin(t f)].
    The argument t*f_i is rounded to fp32 before cos/sin, so compare against float64
    cos/sin of that same fp32 argument.  Plus the reference's own tests: shape, row 0 =
    [1.., 0..], and the base changes the cache (rope.rs:176-258)."""
    R, P = 128, 4096
    cs = oracle.rope_cos_sin_cache(P, R, 1_000_000.0)
    assert cs.shape == (P, R)
    assert np.all(cs[0, :R // 2] == 1.0) and np.all(cs[0, R // 2:] == 0.0)
    i = np.arange(R // 2, dtype=np.float32)
    p32 = np.power(np.float64(1_000_000.0), ((2 * i) / np.float32(R)).astype(np.float64)).astype(np.float32)
    inv = np.float32(1.0) / p32  # powf rounded to fp32, then an fp32 reciprocal
    t = np.arange(P, dtype=np.float32)[:, None]
    arg = (t * inv[None]).astype(np.float32).astype(np.float64)
    np.testing.assert_allclose(cs[:, :R // 2], np.cos(arg), atol=2e-6)
    np.testing.assert_allclose(cs[:, R // 2:], np.sin(arg), atol=2e-6)
    assert not np.allclose(cs, oracle.rope_cos_sin_cache(P, R, 10_000.0))


def _prologue_case(seed, T, Hq, Hkv, D, dtype="bf16", weights=True):
    rng = np.random.default_rng(seed)
    qkv = normal_bits(rng, (T, (Hq + 2 * Hkv) * D), dtype)
    wq = normal_bits(rng, (D,), dtype, 0.1) if weights else None
    wk = normal_bits(rng, (D,), dtype, 0.1) if weights else None
    if weights:  # weights around 1 (trained norms)
        wq = oracle.float_to_half(1.0 + oracle.half_to_float(wq, dtype), dtype)
        wk = oracle.float_to_half(1.0 + oracle.half_to_float(wk, dtype), dtype)
    pos = rng.integers(0, 4096, T).astype(np.int32)
    return qkv, wq, wk, pos


def _numpy_prologue(qkv, Hq, Hkv, D, wq, wk, eps, cs, pos, dtype):
    """Independent vectorised restatement: fp64 mean of squares, float32 division by the
    sqrt, dtype rounding, weight product, then RoPE as (x1 + i x2)(cos + i sin) with every
    product and sum in float32."""
    T = qkv.shape[0]
    x = oracle.half_to_float(qkv[:, :(Hq + Hkv) * D], dtype).reshape(T, Hq + Hkv, D)
    rnd = lambda a: oracle.half_to_float(oracle.float_to_half(a.astype(np.float32), dtype), dtype)  # noqa: E731
    if wq is not None:
        w = np.concatenate([np.repeat(oracle.half_to_float(wq, dtype)[None], Hq, 0),
                            np.repeat(oracle.half_to_float(wk, dtype)[None], Hkv, 0)])[None]
        var = ((x.astype(np.float64) ** 2).sum(-1, keepdims=True)).astype(np.float32) / np.float32(D)
        s = np.sqrt(var + np.float32(eps), dtype=np.float32)
        x = rnd(rnd(x / s) * w)
    c = cs[pos][:, None, :D // 2]
    sn = cs[pos][:, None, D // 2:]
    x1, x2 = x[..., :D // 2], x[..., D // 2:]
    y = np.concatenate([rnd(x1 * c - x2 * sn), rnd(x2 * c + x1 * sn)], -1)
    bits = oracle.float_to_half(y, dtype)
    return bits[:, :Hq], bits[:, Hq:]


@pytest.mark.parametrize("D,dtype,weights", [(128, "bf16", True), (64, "f16", True), (128, "bf16", False)])
def test_prologue_matches_numpy_and_appends(D, dtype, weights):
    T, Hq, Hkv = 9, 4, 2
    qkv, wq, wk, pos = _prologue_case(3, T, Hq, Hkv, D, dtype, weights)
    cs = oracle.rope_cos_sin_cache(4096, D, 1_000_000.0)
    NB, BS = 4, 16
    kc = np.zeros((NB, BS, Hkv, D), np.uint16)
    vc = np.zeros_like(kc)
    slots = np.array([3, 17, -1, 40, 0, 63, 5, 6, 7], np.int64)
    q, k = oracle.qk_norm_rope_and_cache(qkv, Hq, Hkv, D, wq, wk, 1e-6, cs, pos, kc, vc, slots, dtype)
    wq_, wk_ = _numpy_prologue(qkv, Hq, Hkv, D, wq, wk, 1e-6, cs, pos, dtype)
    assert np.array_equal(q, wq_) and np.array_equal(k, wk_)
    kcf, vcf = kc.reshape(-1, Hkv, D), vc.reshape(-1, Hkv, D)
    for t, s in enumerate(slots):
        if s >= 0:
            assert np.array_equal(kcf[s], k[t])
            assert np.array_equal(vcf[s], qkv[t, (Hq + Hkv) * D:].reshape(Hkv, D))
    written = set(int(s) for s in slots if s >= 0)
    assert not kcf[[i for i in range(NB * BS) if i not in written]].any()


def test_prologue_closed_forms():
    """Position 0 is the identity after the norm (the reference's rope test,
    rope.rs:205-223); a constant row with unit weights normalises to 1, and at
    position p the pair (1, 1) turns into (cos - sin, cos + sin); the rotation keeps
    each pair's length."""
    T, Hq, Hkv, D = 4, 2, 1, 128
    cs = oracle.rope_cos_sin_cache(4096, D, 1_000_000.0)
    ones = oracle.float_to_half(np.ones(D, np.float32), "bf16")
    qkv = oracle.float_to_half(np.full((T, (Hq + 2 * Hkv) * D), 3.0, np.float32), "bf16")
    pos = np.array([0, 1, 100, 4095], np.int32)
    q, k = oracle.qk_norm_rope_and_cache(qkv, Hq, Hkv, D, ones, ones, 1e-6, cs, pos)
    qf = oracle.half_to_float(q, "bf16")
    assert np.all(qf[0] == 1.0)
    c, s = cs[pos, :D // 2], cs[pos, D // 2:]
    np.testing.assert_allclose(qf[:, 0, :D // 2], c - s, atol=8e-3)
    np.testing.assert_allclose(qf[:, 0, D // 2:], c + s, atol=8e-3)
    # Random rows: the norm output at position 0 equals the rotated output's pair lengths.
    qkv, wq, wk, _ = _prologue_case(4, 3, Hq, Hkv, D)
    q0, _ = oracle.qk_norm_rope_and_cache(qkv, Hq, Hkv, D, wq, wk, 1e-6, cs, np.zeros(3, np.int32))
    q1, _ = oracle.qk_norm_rope_and_cache(qkv, Hq, Hkv, D, wq, wk, 1e-6, cs, np.array([7, 300, 4000], np.int32))
    a, b = oracle.half_to_float(q0, "bf16"), oracle.half_to_float(q1, "bf16")
    la = np.hypot(a[..., :D // 2], a[..., D // 2:])
    lb = np.hypot(b[..., :D // 2], b[..., D // 2:])
    np.testing.assert_allclose(lb, la, rtol=2e-2, atol=1e-2)


# --------------------------------------------------- committed attention goldens
def test_attention_goldens_reproduce():
    """The committed fixture (tests/golden/attention_goldens.npz, written by
    tests/golden/make_attention_goldens.py from seeded inputs) still equals what the
    fp64 oracle computes: a regression pin of the oracle and of the input generator."""
    import importlib.util

    gold = np.load(Path(__file__).parent / "golden" / "attention_goldens.npz")
    spec = importlib.util.spec_from_file_location("gold", Path(__file__).parent / "golden" / "make_attention_goldens.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert len(gold.files) == len(mod.SPECS)
    for i, sp in enumerate(mod.SPECS):
        q, kc, vc, cuq, cuk, table, scale = mod.case_inputs(sp)
        if sp[0] == "decode":
            o = oracle.paged_decode_attention(q, kc, vc, cuk, table, scale, sp[7], "bf16", use_f64=True)
        else:
            o = oracle.prefill_attention(q, kc, vc, cuq, cuk, scale, table, sp[7], "bf16", use_f64=True)
        np.testing.assert_array_equal(o.astype(np.float32), gold[f"case{i}"], err_msg=f"case{i}")
