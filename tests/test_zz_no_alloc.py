"""paged_decode_attention_noalloc (partials in the library's static device scratch)
against the workspace entry points, called through the C ABI: bit-identical
output and caches on two calls in a row, the second with a smaller input (the
scratch still holds the first call's partials), with and without the fused
append, windowed and not; a shape beyond the scratch is rejected before any
launch."""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _step(cfg_id, seed, device):
    import torch
    from oxide_paged_kv.workload import CONFIGS, make_decode_step

    st = make_decode_step(CONFIGS[cfg_id], seed=seed)
    c = st.cfg
    g = torch.Generator(device=device).manual_seed(seed)
    shape = (st.pool_blocks, c.block_size, c.num_kv_heads, c.head_dim)
    kc = torch.randn(shape, generator=g, device=device).bfloat16()
    vc = torch.randn(shape, generator=g, device=device).bfloat16()
    q = torch.randn((c.batch, c.num_heads, c.head_dim), generator=g, device=device).bfloat16()
    kn = torch.randn((c.batch, c.num_kv_heads, c.head_dim), generator=g, device=device).bfloat16()
    vn = torch.randn((c.batch, c.num_kv_heads, c.head_dim), generator=g, device=device).bfloat16()
    meta = (torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device), torch.from_numpy(st.block_table).to(device))
    return st, kc, vc, q, (kn, vn, torch.from_numpy(st.slot_mapping).to(device)), meta


def _same(a, b):
    import torch

    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("order", [(3, 1), (5, 4)], ids=["cfg3-then-cfg1", "cfg5-then-cfg4"])
def test_noalloc_matches_workspace_entry(device, order):
    import torch
    import oxide_paged_kv as ox

    for cfg_id in order:  # the second call is the smaller input
        st, kc, vc, q, app, (cu, bt) = _step(cfg_id, 100 + cfg_id, device)
        c = st.cfg
        w = None if c.window_left < 0 else c.window_left
        scale = 1 / math.sqrt(c.head_dim)
        print(f"noalloc cfg{cfg_id} B={c.batch} window={c.window_left} "
              f"split_tokens={ox.split_tokens(c.batch, c.num_kv_heads, st.max_seqlen_k)}", flush=True)
        k2, v2 = kc.clone(), vc.clone()
        want = ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale, w, append=app)
        got = ox.decode_attn(q, k2, v2, cu, bt, st.max_seqlen_k, scale, w, append=app, noalloc=True)
        torch.cuda.synchronize()
        assert _same(got, want)
        assert _same(k2, kc) and _same(v2, vc)
        want = ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale, w)
        got = ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale, w, noalloc=True)
        torch.cuda.synchronize()
        assert _same(got, want)
        del kc, vc, k2, v2
        torch.cuda.empty_cache()


def test_noalloc_rejects_shape_beyond_scratch(device):
    """15 sequences of 65536 keys at 128 query heads over 8 kv heads take the split grid
    with 1024-key splits: 122,880 partial rows of 512 B = 60 MiB > 48 MiB."""
    import torch
    import oxide_paged_kv as ox
    from oxide_paged_kv import _lib

    B, Hq, Hkv, D, L = 15, 128, 8, 128, 65536
    assert ox.split_tokens(B, Hkv, L) == 1024
    q = torch.zeros((B, Hq, D), dtype=torch.bfloat16, device=device)
    kc = torch.zeros((1, 256, Hkv, D), dtype=torch.bfloat16, device=device)
    out = torch.full_like(q, 7.0)
    cu = torch.arange(B + 1, dtype=torch.int32, device=device) * L
    bt = torch.zeros((B, L // 256), dtype=torch.int32, device=device)
    with pytest.raises(_lib.OxideError, match="error 5"):
        ox.decode_attn(q, kc, kc, cu, bt, L, 1 / math.sqrt(D), out=out, noalloc=True)
    torch.cuda.synchronize()
    assert bool((out.float() == 7.0).all())  # nothing was launched


def test_noalloc_under_graph_capture(device):
    """The allocation-free entry captured into a HIP graph (torch.cuda.CUDAGraph on the
    capture stream): the fused append + attention on a cfg3-sized batch and a plain call on
    a small one; the graph is replayed three times with eager calls of the workspace entry
    and host synchronisations in between, and every replay's output and caches must equal
    the eager result bit for bit."""
    import torch
    import oxide_paged_kv as ox

    st, kc, vc, q, app, (cu, bt) = _step(3, 200, device)
    c = st.cfg
    scale = 1 / math.sqrt(c.head_dim)
    st1, kc1, vc1, q1, _, (cu1, bt1) = _step(1, 201, device)
    scale1 = 1 / math.sqrt(st1.cfg.head_dim)
    # Eager references: the append is idempotent (same rows to the same slots).
    k_ref, v_ref = kc.clone(), vc.clone()
    want = ox.decode_attn(q, k_ref, v_ref, cu, bt, st.max_seqlen_k, scale, append=app)
    want1 = ox.decode_attn(q1, kc1, vc1, cu1, bt1, st1.max_seqlen_k, scale1)
    out = torch.empty_like(q)
    out1 = torch.empty_like(q1)
    # Warm up on the side stream the capture will use (first-call device queries).
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale, out=out, append=app, noalloc=True)
        ox.decode_attn(q1, kc1, vc1, cu1, bt1, st1.max_seqlen_k, scale1, out=out1, noalloc=True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale, out=out, append=app, noalloc=True)
        ox.decode_attn(q1, kc1, vc1, cu1, bt1, st1.max_seqlen_k, scale1, out=out1, noalloc=True)
    for rep in range(3):
        out.fill_(0)
        out1.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        print(f"graph replay {rep}", flush=True)
        assert _same(out, want) and _same(out1, want1), rep
        assert _same(kc, k_ref) and _same(vc, v_ref), rep
        # eager work between the replays, on the default stream
        ox.decode_attn(q1, kc1, vc1, cu1, bt1, st1.max_seqlen_k, scale1)
        torch.cuda.synchronize()


_CAPTURE_FIRST = r'''
import math, sys
sys.path[:0] = [{repo!r}, {pkg!r}]
import numpy as np
import torch
import oxide_paged_kv as ox
from oxide_paged_kv.workload import CONFIGS, make_decode_step

dev = torch.device("cuda:0")
st = make_decode_step(CONFIGS[{cfg}], seed=300)
c = st.cfg
g = torch.Generator(device=dev).manual_seed(300)
shape = (st.pool_blocks, c.block_size, c.num_kv_heads, c.head_dim)
kc = torch.randn(shape, generator=g, device=dev).bfloat16()
vc = torch.randn(shape, generator=g, device=dev).bfloat16()
q = torch.randn((c.batch, c.num_heads, c.head_dim), generator=g, device=dev).bfloat16()
cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(dev)
bt = torch.from_numpy(st.block_table).to(dev)
scale = 1 / math.sqrt(c.head_dim)
out = torch.empty_like(q)
ox.load()  # the library is loaded (its code objects registered) before the capture
torch.cuda.synchronize()
# The library's first call in this process is the one being captured.
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale, out=out, noalloc=True)
for rep in range(2):
    out.fill_(0)
    graph.replay()
    torch.cuda.synchronize()
    want = ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16)), rep
print("capture-first ok", flush=True)
'''


@pytest.mark.parametrize("cfg_id", [1, 3], ids=["split-grid-cfg1", "stream-cfg3"])
def test_noalloc_first_call_under_graph_capture(cfg_id):
    """In a fresh process whose first library call is the allocation-free entry under
    HIP graph capture (no warm-up: the device queries and the scratch address lookup
    run during the capture), the replays equal the workspace entry bit for bit."""
    import subprocess
    import sys
    from pathlib import Path

    repo = Path(__file__).resolve().parent.parent
    code = _CAPTURE_FIRST.format(repo=str(repo), pkg=str(repo / "vllm-oxide_amd"), cfg=cfg_id)
    print(f"capture-first subprocess cfg{cfg_id}", flush=True)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and "capture-first ok" in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]
