"""Writes tests/golden/attention_goldens.npz: fp64-oracle outputs of paged decode and
prefill attention on small seeded cases (<= 4 sequences, <= 3 blocks, D = 128,
G in {1, 2, 4, 8}, window none or 100).

The inputs are not stored: `case_inputs(spec)` regenerates them from the spec's seed
with numpy's PCG64 generator (bit-reproducible across platforms), so the fixture is
only the expected outputs.  Run from the repository root after building the oracle:
    python tests/golden/make_attention_goldens.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))
sys.path.insert(0, str(REPO / "tests"))

OUT = Path(__file__).resolve().parent / "attention_goldens.npz"

# kind, seed, G, Hkv, block_size, lq (prefill), lens (keys), window
SPECS = [
    ("decode", 1, 1, 2, 256, None, [300, 1, 700, 0], -1),
    ("decode", 2, 2, 2, 256, None, [768, 257, 5], 100),
    ("decode", 3, 4, 2, 256, None, [513, 100, 99, 768], -1),
    ("decode", 4, 8, 1, 256, None, [640, 2], 100),
    ("prefill", 5, 1, 2, 256, [12, 7], [300, 7], -1),
    ("prefill", 6, 2, 2, 256, [9, 1, 5], [64, 600, 40], 100),
    ("prefill", 7, 4, 2, 256, [6, 11], [700, 50], -1),
    ("prefill", 8, 8, 1, 256, [5], [517], 100),
]
D = 128


def case_inputs(spec):
    """(q, k_cache, v_cache, cu_seqlens_q | None, cu_seqlens_k, block_table, scale) as uint16
    bit patterns of bf16, regenerated from the spec."""
    from helpers import normal_bits

    kind, seed, G, Hkv, BS, lq, lens, window = spec
    rng = np.random.Generator(np.random.PCG64(seed))
    lens = np.asarray(lens, np.int64)
    nblk = (lens + BS - 1) // BS
    NB = int(nblk.sum()) + 1
    perm = rng.permutation(NB).astype(np.int32)
    table = np.zeros((len(lens), max(int(nblk.max()), 1)), np.int32)
    pos = 0
    for b in range(len(lens)):
        table[b, :nblk[b]] = perm[pos:pos + nblk[b]]
        pos += nblk[b]
    cuk = np.zeros(len(lens) + 1, np.uint32)
    cuk[1:] = np.cumsum(lens)
    Hq = G * Hkv
    kc = normal_bits(rng, (NB, BS, Hkv, D))
    vc = normal_bits(rng, (NB, BS, Hkv, D))
    if kind == "decode":
        q = normal_bits(rng, (len(lens), Hq, D))
        cuq = None
    else:
        cuq = np.zeros(len(lq) + 1, np.uint32)
        cuq[1:] = np.cumsum(lq)
        q = normal_bits(rng, (int(cuq[-1]), Hq, D))
    return q, kc, vc, cuq, cuk, table, 1.0 / np.sqrt(D)


def main() -> None:
    import oracle

    outs = {}
    for i, spec in enumerate(SPECS):
        q, kc, vc, cuq, cuk, table, scale = case_inputs(spec)
        window = spec[7]
        if spec[0] == "decode":
            o = oracle.paged_decode_attention(q, kc, vc, cuk, table, scale, window, "bf16", use_f64=True)
        else:
            o = oracle.prefill_attention(q, kc, vc, cuq, cuk, scale, table, window, "bf16", use_f64=True)
        outs[f"case{i}"] = o.astype(np.float32)
    np.savez_compressed(OUT, **outs)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(outs)} cases)")


if __name__ == "__main__":
    main()
