"""Benchmark configuration 2 at full size: Qwen3-0.6B decode shape (16 q / 8 kv heads,
D 128, bf16, block 256), batch 32, context U[512, 4096], a 4096-block pool,
through the per-layer views of the reference's 28-layer buffer
[2, 28, 4096, 256, 8, 128] (PagedKVCache::new / k_cache / v_cache,
crates/vllm-oxide/src/attention/mod.rs:55-85; kv_cache_layout_shape,
crates/vllm-oxide/src/utils.rs:46-61).

On three layers (first, middle, last): the fused append + decode attention
equals reshape_and_cache followed by paged_decode_attention bit for bit
(output and caches), sampled sequences match the oracle (target tolerance and
the output-scaled bar), and the neighbouring layers' views are untouched.
"""
import math

import numpy as np
import pytest

import oracle
from helpers import assert_attn_close, assert_attn_scaled, to_bits, to_f32

pytestmark = pytest.mark.gpu


def test_decode_cfg2_full_size_per_layer_views(device):
    import torch
    import oxide_paged_kv as ox
    from oxide_paged_kv.workload import CONFIGS, make_decode_step

    cfg = CONFIGS[2]
    st = make_decode_step(cfg, seed=22)
    NL, NB, BS, H, D = cfg.layers, st.pool_blocks, cfg.block_size, cfg.num_kv_heads, cfg.head_dim
    assert (NL, NB) == (28, 4096)
    print(f"cfg2 buffer [2, {NL}, {NB}, {BS}, {H}, {D}] bf16 = {2 * NL * NB * BS * H * D * 2 / 2**30:.0f} GiB",
          flush=True)
    g = torch.Generator(device=device).manual_seed(22)
    buf = torch.empty((2, NL, NB, BS, H, D), dtype=torch.bfloat16, device=device)
    for kv in range(2):
        for layer in range(NL):
            buf[kv, layer].normal_(generator=g)
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(device)
    bt = torch.from_numpy(st.block_table).to(device)
    sm = torch.from_numpy(st.slot_mapping).to(device)
    scale = 1 / math.sqrt(D)
    assert ox.split_tokens(cfg.batch, H, st.max_seqlen_k) > 0  # the shape policy picks the split grid
    lens = st.context_lens.astype(np.int64)
    samples = sorted({int(lens.argmax()), int(lens.argmin()), 0, cfg.batch - 1})
    slots = st.slot_mapping
    blk_new, off_new = torch.from_numpy(slots // BS).to(device), torch.from_numpy(slots % BS).to(device)
    for layer in (0, 13, 27):
        print(f"cfg2 layer {layer}", flush=True)
        q = torch.randn((cfg.batch, cfg.num_heads, D), generator=g, device=device).bfloat16()
        kn = torch.randn((cfg.batch, H, D), generator=g, device=device).bfloat16()
        vn = torch.randn((cfg.batch, H, D), generator=g, device=device).bfloat16()
        kc, vc = buf[0, layer], buf[1, layer]  # the reference's per-layer views
        assert kc.data_ptr() == buf.data_ptr() + layer * NB * BS * H * D * 2
        assert vc.data_ptr() == buf.data_ptr() + (NL + layer) * NB * BS * H * D * 2
        neighbours = [buf[kv, n][blk_new, off_new].clone() for kv in range(2) for n in (layer - 1, layer + 1)
                      if 0 <= n < NL]
        k2, v2 = kc.clone(), vc.clone()
        got = ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale, append=(kn, vn, sm))
        ox.reshape_and_cache(kn, vn, k2, v2, sm)
        want = ox.decode_attn(q, k2, v2, cu, bt, st.max_seqlen_k, scale)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        assert torch.equal(kc.view(torch.int16), k2.view(torch.int16))
        assert torch.equal(vc.view(torch.int16), v2.view(torch.int16))
        assert torch.equal(kc[blk_new, off_new].view(torch.int16), kn.view(torch.int16))
        after = [buf[kv, n][blk_new, off_new] for kv in range(2) for n in (layer - 1, layer + 1) if 0 <= n < NL]
        for a, b in zip(neighbours, after):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16))
        del k2, v2
        out = to_f32(got)
        for b in samples:
            ids = torch.from_numpy(np.asarray(st.block_rows[b], np.int64)).to(device)
            ref = oracle.paged_decode_attention(
                to_bits(q[b:b + 1]), to_bits(kc[ids]), to_bits(vc[ids]), np.array([0, lens[b]], np.uint32),
                np.arange(len(ids), dtype=np.int32)[None], scale, -1, threads=16)
            assert_attn_close(out[b:b + 1], ref)
            assert_attn_scaled(out[b:b + 1], ref, label=f"cfg2 layer {layer} seq {b} L={lens[b]}")
    del buf
    torch.cuda.empty_cache()
