"""paged_decode_attention_shared_prefix (cascaded decode over a shared block-table
prefix) against the oracle and against the plain entries.

The cascade attends the leading block-table entries that every row shares once
for the whole batch (matrix cores) and the remaining keys per sequence (the stream
pass), then merges both; the shared count is found on the device, the caller's
hint being an upper bound.  Cases cover exact, too large and zero hints, rows that
diverge early, a sequence shorter than the shared prefix, an empty sequence (no
cascade), windows that start inside and past the prefix, page sizes 16 / 64 / 256,
groups 1 / 2 / 4 / 8 / 16, D 64 / 128, f16 and bf16, the fused append (bit-identical
cache, the new token attended), and the full-size cfg4 step through both entries.
Every case runs through both forms of the cascade, forced (the two passes one after the
other, and the prefix pass beside the stream pass on the library's side stream): by
shape these batches save too few bytes and would run the plain entries; the cfg4 test
runs the form chosen by shape (overlapped).  Both passes find the shared count
themselves.
Tolerance: the target's (max-abs 2e-2, max-rel 1e-2) and the output-scaled bar.
"""
import math

import numpy as np
import pytest

import oracle
from helpers import assert_attn_close, assert_attn_scaled, normal_bits, to_bits, to_f32, to_torch

pytestmark = pytest.mark.gpu


def _shared_case(seed, B, Hq, Hkv, D, BS, shared, extra, dtype="bf16", diverge=None):
    """B sequences of L_b = shared * BS + extra[b] keys (extra may be negative: a
    sequence shorter than the shared prefix, or empty) whose first `shared` blocks (as
    far as they reach) are the same block ids, then private blocks.  diverge: {b: j}
    gives row b a private block id at entry j < shared instead."""
    rng = np.random.default_rng(seed)
    extra = np.asarray(extra, np.int64)
    lens = shared * BS + extra
    assert (lens >= 0).all()
    priv = np.maximum((lens - shared * BS + BS - 1) // BS, 0)
    NB = shared + int(priv.sum()) + B + 8
    perm = rng.permutation(NB).astype(np.int32)
    common = perm[:shared]
    pos = shared
    width = max(int(((lens + BS - 1) // BS).max()), shared, 1)
    table = np.zeros((B, width), np.int32)
    for b in range(B):
        nb = int((lens[b] + BS - 1) // BS)
        row = list(common[:min(shared, nb)])
        for _ in range(nb - len(row)):
            row.append(perm[pos])
            pos += 1
        if diverge and b in diverge and diverge[b] < len(row):
            row[diverge[b]] = perm[pos]
            pos += 1
        table[b, :len(row)] = row
    assert pos <= NB
    cu = np.zeros(B + 1, np.uint32)
    cu[1:] = np.cumsum(lens)
    q = normal_bits(rng, (B, Hq, D), dtype)
    kc = normal_bits(rng, (NB, BS, Hkv, D), dtype)
    vc = normal_bits(rng, (NB, BS, Hkv, D), dtype)
    return q, kc, vc, cu, table, int(lens.max()), lens


CASES = [
    # (B, Hq, Hkv, D, BS, shared, extra, window, hint, dtype, diverge)
    (6, 32, 8, 128, 256, 3, [1, 5, 300, 256, 700, 64], -1, 3, "bf16", None),      # exact hint
    (6, 32, 8, 128, 256, 3, [1, 5, 300, 256, 700, 64], -1, 8, "bf16", None),      # hint too large
    (6, 32, 8, 128, 256, 3, [1, 5, 300, 256, 700, 64], 500, 3, "bf16", None),     # window inside prefix
    (6, 32, 8, 128, 256, 3, [1, 5, 300, 256, 700, 64], 100, 3, "bf16", None),     # window past prefix
    (5, 16, 8, 128, 64, 6, [10, 1, 200, 64, 33], -1, 6, "f16", {3: 2}),          # a row diverges at 2
    (5, 16, 8, 128, 16, 20, [3, 17, 40, 1, 100], 37, 25, "bf16", None),           # BS 16, window
    (4, 8, 8, 128, 256, 2, [-512, 100, 300, 1], -1, 2, "bf16", None),             # empty sequence
    (5, 32, 8, 128, 256, 4, [30, -300, 500, 0, 9], 2000, 4, "bf16", None),        # short sequence, L = 4 BS
    (4, 64, 8, 128, 256, 4, [1, 800, 9, 2000], -1, 4, "bf16", None),              # G 8
    (3, 4, 2, 64, 64, 5, [70, 1, 129], 200, 5, "f16", None),                      # G 2, D 64
    (3, 32, 2, 64, 32, 6, [5, 90, 33], -1, 6, "bf16", None),                      # G 16
    (130, 32, 8, 128, 256, 2, list(range(1, 131)), -1, 2, "bf16", None),          # 2 row tiles
    # Longer private parts (by shape the overlap would be chosen if the batch saved
    # enough bytes to take the cascade at all):
    (32, 32, 8, 128, 256, 4, [4096 - 97 * i for i in range(30)] + [-1024, -500], -1, 4, "bf16", None),
    (32, 32, 8, 128, 256, 4, [4096 - 97 * i for i in range(30)] + [-1024, -500], 3000, 6, "f16", {5: 1}),
    (16, 64, 8, 128, 256, 3, [8000 - 333 * i for i in range(16)], -1, 3, "bf16", None),             # G 8
    (24, 32, 8, 128, 64, 12, [5000 + 5 * i for i in range(24)], 1500, 12, "bf16", {0: 11}),        # BS 64
]


def _run(device, case, append, mode="auto"):
    import torch
    import oxide_paged_kv as ox

    B, Hq, Hkv, D, BS, shared, extra, window, hint, dtype, diverge = case
    q, kc, vc, cu, table, mx, lens = _shared_case(7, B, Hq, Hkv, D, BS, shared, extra, dtype, diverge)
    scale = 1 / math.sqrt(D)
    t = lambda a: to_torch(a, dtype, device)  # noqa: E731
    cu_d = torch.from_numpy(cu.view(np.int32)).to(device)
    bt_d = torch.from_numpy(table).to(device)
    w = None if window < 0 else window
    kc2, vc2 = kc.copy(), vc.copy()
    app = None
    if append:
        rng = np.random.default_rng(11)
        kn, vn = normal_bits(rng, (B, Hkv, D), dtype), normal_bits(rng, (B, Hkv, D), dtype)
        NB = kc.shape[0]
        used = {int(x) for x in table.ravel()}
        spare = [blk for blk in range(NB) if blk not in used]
        slots = np.array([table[b, (L - 1) // BS] * BS + (L - 1) % BS if L > 0 else spare[b % len(spare)] * BS
                          for b, L in enumerate(lens)], np.int64)
        # A new token whose block other rows also hold skips its append (-1): an engine
        # copies such a block first, and the fused append assumes no other sequence
        # reads the slot it writes.
        holders = {}
        for b, L in enumerate(lens):
            for x in set(int(v) for v in table[b, :(L + BS - 1) // BS]):
                holders[x] = holders.get(x, 0) + 1
        for b, L in enumerate(lens):
            if L > 0 and holders[int(table[b, (L - 1) // BS])] > 1:
                slots[b] = -1
        oracle.reshape_and_cache(kn, vn, kc2, vc2, slots)
        app = (t(kn), t(vn), torch.from_numpy(slots).to(device))
    want = oracle.paged_decode_attention(q, kc2, vc2, cu, table, scale, window, dtype)
    kd, vd = t(kc), t(vc)
    got = ox.decode_attn(t(q), kd, vd, cu_d, bt_d, mx, scale, w, BS, append=app, shared_prefix_blocks=hint,
                         shared_prefix_mode=mode)
    torch.cuda.synchronize()
    return to_f32(got), want, (to_bits(kd), to_bits(vd)), (kc2, vc2)


@pytest.mark.parametrize("case", CASES, ids=[f"s{i}" for i in range(len(CASES))])
@pytest.mark.parametrize("append", [False, True], ids=["plain", "append"])
@pytest.mark.parametrize("mode", ["serial", "overlap"])
def test_cascade_vs_oracle(device, case, append, mode):
    """Every case through both forms of the cascade, forced (by shape most of these small
    batches would run the plain entries: the cascade saves them too few bytes)."""
    print(f"cascade case {case[:7]} window={case[7]} hint={case[8]} {case[9]} append={append} {mode}", flush=True)
    got, want, caches, want_caches = _run(device, case, append, mode)
    assert_attn_close(got, want)
    assert_attn_scaled(got, want, label=f"cascade {case[:5]}")
    if append:
        assert np.array_equal(caches[0], want_caches[0]) and np.array_equal(caches[1], want_caches[1])


def _random_cases(n, seed):
    """Seeded random shapes: kv heads 1 / 2 / 4 / 8, groups 1 / 2 / 4 / 8 / 16, D 64 / 128,
    pages 16 / 32 / 64 / 256, ragged lengths (some shorter than the shared prefix, some
    empty), a window on half of them, an oversized hint on some, a diverging row on some."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        Hkv = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.choice([1, 2, 4, 8, 16]))
        D = int(rng.choice([64, 128]))
        BS = int(rng.choice([16, 32, 64, 256]))
        B = int(rng.integers(2, 40))
        shared = int(rng.integers(1, max(2, 2048 // BS)))
        extra = [int(x) for x in rng.integers(-shared * BS // 2, 900, size=B)]
        if B > 3:
            extra[int(rng.integers(0, B))] = -shared * BS  # an empty sequence
        window = int(rng.integers(10, 2500)) if rng.random() < 0.5 else -1
        hint = shared + int(rng.integers(0, 3))
        diverge = {int(rng.integers(1, B)): int(rng.integers(0, shared))} if rng.random() < 0.3 else None
        dtype = "bf16" if rng.random() < 0.7 else "f16"
        out.append((B, G * Hkv, Hkv, D, BS, shared, extra, window, hint, dtype, diverge))
    return out


RANDOM_CASES = _random_cases(12, 2024)


@pytest.mark.parametrize("case", RANDOM_CASES, ids=[f"r{i}" for i in range(len(RANDOM_CASES))])
@pytest.mark.parametrize("mode", ["serial", "overlap"])
def test_cascade_random_shapes(device, case, mode):
    print(f"cascade random case {case[:7]} window={case[7]} hint={case[8]} {case[9]} {mode}", flush=True)
    got, want, _, _ = _run(device, case, False, mode)
    assert_attn_close(got, want)
    assert_attn_scaled(got, want, label=f"cascade random {case[:5]}")


def test_cascade_plan_by_shape(device):
    """The by-shape form: the plain entries where the cascade saves under 200 MB of K/V
    reads (small batches), the cascade beyond, overlapped when the per-sequence part is long
    (cfg4); shapes the stream pass does not take always run the plain entries.  A batch the
    plan sends to the plain entries gives the plain entry's bits."""
    import torch
    import oxide_paged_kv as ox

    assert ox.shared_prefix_plan(4, 32, 8, 128, 256, 8192 + 256, 32) == "plain"
    assert ox.shared_prefix_plan(16, 32, 8, 128, 256, 2048 + 1024, 8) == "plain"
    assert ox.shared_prefix_plan(32, 32, 8, 128, 256, 4096 + 2000, 16) != "plain"
    assert ox.shared_prefix_plan(128, 32, 8, 128, 256, 5120, 16) == "overlap"
    assert ox.shared_prefix_plan(128, 32, 6, 128, 256, 5120, 16) == "plain"  # kv heads not dividing 8
    assert ox.shared_prefix_plan(128, 32, 8, 128, 256, 5120, 0) == "plain"
    case = CASES[0]
    B, Hq, Hkv, D, BS, shared, extra, window, hint, dtype, diverge = case
    assert ox.shared_prefix_plan(B, Hq, Hkv, D, BS, shared * BS + max(extra), hint) == "plain"
    q, kc, vc, cu, table, mx, lens = _shared_case(3, B, Hq, Hkv, D, BS, shared, extra, dtype, diverge)
    t = lambda a: to_torch(a, dtype, device)  # noqa: E731
    args = (t(q), t(kc), t(vc), torch.from_numpy(cu.view(np.int32)).to(device), torch.from_numpy(table).to(device),
            mx, 1 / math.sqrt(D), None, BS)
    a = to_bits(ox.decode_attn(*args, shared_prefix_blocks=hint))
    b = to_bits(ox.decode_attn(*args))
    torch.cuda.synchronize()
    assert np.array_equal(a, b)


def test_cascade_hint_zero_is_the_plain_entry(device):
    """A hint of 0 runs the plain entry: bit-identical output."""
    import torch
    import oxide_paged_kv as ox

    q, kc, vc, cu, table, mx, lens = _shared_case(3, 4, 32, 8, 128, 256, 2, [3, 400, 1, 90])
    t = lambda a: to_torch(a, "bf16", device)  # noqa: E731
    args = (t(q), t(kc), t(vc), torch.from_numpy(cu.view(np.int32)).to(device), torch.from_numpy(table).to(device),
            mx, 1 / math.sqrt(128))
    a = to_bits(ox.decode_attn(*args, shared_prefix_blocks=0))
    b = to_bits(ox.decode_attn(*args))
    torch.cuda.synchronize()
    assert np.array_equal(a, b)


@pytest.mark.parametrize("fused", [True, False], ids=["fused-append", "plain"])
def test_cascade_cfg4_full_size(device, fused):
    """Full-size cfg4 (128 sequences sharing 15 prefix blocks after the copy-on-write
    of the 16th, window 4096): the cascade against the plain entry (stream pass) on
    the same inputs -- outputs within the attention tolerance and the scaled bar, the
    fused append's cache bit-identical -- and two sequences against the oracle."""
    import torch
    import oxide_paged_kv as ox
    from oxide_paged_kv.workload import CONFIGS, make_decode_step

    st = make_decode_step(CONFIGS[4], seed=44)
    c = st.cfg
    g = torch.Generator(device=device).manual_seed(44)
    shape = (st.pool_blocks, c.block_size, c.num_kv_heads, c.head_dim)
    kc = torch.randn(shape, generator=g, device=device).bfloat16()
    vc = torch.randn(shape, generator=g, device=device).bfloat16()
    pairs = torch.from_numpy(st.cow_pairs).to(device)
    ox.copy_blocks(kc, vc, pairs)
    q = torch.randn((c.batch, c.num_heads, c.head_dim), generator=g, device=device).bfloat16()
    kn = torch.randn((c.batch, c.num_kv_heads, c.head_dim), generator=g, device=device).bfloat16()
    vn = torch.randn((c.batch, c.num_kv_heads, c.head_dim), generator=g, device=device).bfloat16()
    sm = torch.from_numpy(st.slot_mapping).to(device)
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device)
    bt = torch.from_numpy(st.block_table).to(device)
    scale = 1 / math.sqrt(c.head_dim)
    hint = c.shared_prefix // c.block_size
    k1, v1, k2, v2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    app1 = (kn, vn, sm) if fused else None
    if not fused:
        ox.reshape_and_cache(kn, vn, k1, v1, sm)
        ox.reshape_and_cache(kn, vn, k2, v2, sm)
    want = ox.decode_attn(q, k1, v1, cu, bt, st.max_seqlen_k, scale, c.window_left, append=app1)
    got = ox.decode_attn(q, k2, v2, cu, bt, st.max_seqlen_k, scale, c.window_left, append=app1,
                         shared_prefix_blocks=hint)
    torch.cuda.synchronize()
    assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
    assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))
    g_np, w_np = to_f32(got), to_f32(want)
    assert_attn_close(g_np, w_np)
    assert_attn_scaled(g_np, w_np, label="cfg4 cascade vs stream")
    lens = st.context_lens.astype(np.int64)
    for b in (int(lens.argmax()), int(lens.argmin())):
        ids = torch.from_numpy(np.asarray(st.block_rows[b], np.int64)).to(device)
        ref = oracle.paged_decode_attention(to_bits(q[b:b + 1]), to_bits(k2[ids]), to_bits(v2[ids]),
                                            np.array([0, lens[b]], np.uint32),
                                            np.arange(len(ids), dtype=np.int32)[None], scale, c.window_left,
                                            threads=16)
        assert_attn_close(g_np[b:b + 1], ref)


def test_cascade_overlapped_under_graph_capture(device):
    """An overlapped cascaded call (prefix pass forked onto the library's side stream and
    joined back) captured into a HIP graph on torch's capture stream: three replays with
    eager cascaded calls and host synchronisations between them, each replay's output
    bit-identical to the eager call on the same inputs."""
    import torch
    import oxide_paged_kv as ox

    case = CASES[12]
    B, Hq, Hkv, D, BS, shared, extra, window, hint, dtype, diverge = case
    q, kc, vc, cu, table, mx, lens = _shared_case(21, B, Hq, Hkv, D, BS, shared, extra, dtype, diverge)
    t = lambda a: to_torch(a, dtype, device)  # noqa: E731
    cu_d = torch.from_numpy(cu.view(np.int32)).to(device)
    bt_d = torch.from_numpy(table).to(device)
    qd, kd, vd = t(q), t(kc), t(vc)
    scale = 1 / math.sqrt(D)
    ws = torch.zeros(ox.shared_prefix_workspace_size(B, Hq, Hkv, D, BS, mx, hint), dtype=torch.uint8, device=device)
    kw = dict(shared_prefix_blocks=hint, shared_prefix_mode="overlap")
    want = ox.decode_attn(qd, kd, vd, cu_d, bt_d, mx, scale, None, BS, **kw)
    out = torch.empty_like(qd)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm-up on the stream the capture will use
        ox.decode_attn(qd, kd, vd, cu_d, bt_d, mx, scale, None, BS, out=out, workspace=ws, **kw)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ox.decode_attn(qd, kd, vd, cu_d, bt_d, mx, scale, None, BS, out=out, workspace=ws, **kw)
    for rep in range(3):
        out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        print(f"cascade graph replay {rep}", flush=True)
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), rep
        ox.decode_attn(qd, kd, vd, cu_d, bt_d, mx, scale, None, BS, **kw)
        torch.cuda.synchronize()
    got = to_f32(out)
    ref = oracle.paged_decode_attention(q, kc, vc, cu, table, scale, window, dtype)
    assert_attn_close(got, ref)


def test_cascade_overlapped_from_two_threads(device):
    """Overlapped cascaded calls from two host threads at once, each on its own stream
    (each thread forks onto its own side stream): every call's output bit-identical to
    the same call made alone."""
    import threading

    import torch
    import oxide_paged_kv as ox

    case = CASES[12]
    B, Hq, Hkv, D, BS, shared, extra, window, hint, dtype, diverge = case
    q, kc, vc, cu, table, mx, lens = _shared_case(31, B, Hq, Hkv, D, BS, shared, extra, dtype, diverge)
    t = lambda a: to_torch(a, dtype, device)  # noqa: E731
    cu_d = torch.from_numpy(cu.view(np.int32)).to(device)
    bt_d = torch.from_numpy(table).to(device)
    kd, vd = t(kc), t(vc)
    qs = [t(q), t(q[::-1].copy())]
    kw = dict(shared_prefix_blocks=hint, shared_prefix_mode="overlap")
    scale = 1 / math.sqrt(D)
    want = [ox.decode_attn(qq, kd, vd, cu_d, bt_d, mx, scale, None, BS, **kw) for qq in qs]
    torch.cuda.synchronize()
    outs = [[None] * 5 for _ in range(2)]
    errors = []

    def work(i):
        try:
            s = torch.cuda.Stream()
            ws = torch.zeros(ox.shared_prefix_workspace_size(B, Hq, Hkv, D, BS, mx, hint), dtype=torch.uint8,
                             device=device)
            with torch.cuda.stream(s):
                for r in range(5):
                    outs[i][r] = ox.decode_attn(qs[i], kd, vd, cu_d, bt_d, mx, scale, None, BS, workspace=ws, **kw)
            s.synchronize()
        except Exception as e:  # noqa: BLE001 -- reported below
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    for i in range(2):
        for r in range(5):
            assert torch.equal(outs[i][r].view(torch.int16), want[i].view(torch.int16)), (i, r)


_CASCADE_CAPTURE_FIRST = r'''
import math, sys
sys.path[:0] = [{repo!r}, {pkg!r}, {tests!r}]
import numpy as np
import torch
import oxide_paged_kv as ox
import test_gpu_decode_cascade as T
from helpers import to_torch

dev = torch.device("cuda:0")
B, Hq, Hkv, D, BS, shared, extra, window, hint, dtype, diverge = T.CASES[12]
q, kc, vc, cu, table, mx, lens = T._shared_case(41, B, Hq, Hkv, D, BS, shared, extra, dtype, diverge)
t = lambda a: to_torch(a, dtype, dev)
qd, kd, vd = t(q), t(kc), t(vc)
cu_d = torch.from_numpy(cu.view(np.int32)).to(dev)
bt_d = torch.from_numpy(table).to(dev)
ws = torch.zeros(ox.shared_prefix_workspace_size(B, Hq, Hkv, D, BS, mx, hint), dtype=torch.uint8, device=dev)
out = torch.empty_like(qd)
kw = dict(shared_prefix_blocks=hint, shared_prefix_mode="overlap")
ox.load()
torch.cuda.synchronize()
# The library's first call in this process -- the one that creates the side stream -- is captured.
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    ox.decode_attn(qd, kd, vd, cu_d, bt_d, mx, 1 / math.sqrt(D), None, BS, out=out, workspace=ws, **kw)
for rep in range(2):
    out.fill_(0)
    graph.replay()
    torch.cuda.synchronize()
    want = ox.decode_attn(qd, kd, vd, cu_d, bt_d, mx, 1 / math.sqrt(D), None, BS, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16)), rep
print("cascade capture-first ok", flush=True)
'''


def test_cascade_first_call_under_graph_capture():
    """In a fresh process whose first library call is an overlapped cascaded call under HIP
    graph capture (the side stream and its events are created during the capture), the
    replays equal the eager call bit for bit."""
    import subprocess
    import sys
    from pathlib import Path

    repo = Path(__file__).resolve().parent.parent
    code = _CASCADE_CAPTURE_FIRST.format(repo=str(repo), pkg=str(repo / "vllm-oxide_amd"), tests=str(repo / "tests"))
    print("cascade capture-first subprocess", flush=True)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and "cascade capture-first ok" in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]
