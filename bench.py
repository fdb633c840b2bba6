"""Benchmark of the paged-KV decode hot path on one MI355X.

A step is one layer's decode-time work on the paged cache, in the reference's
order (models/qwen3.rs:199-208): KV append of one new token per sequence
(reshape_and_cache), then paged decode attention over every sequence's context --
by default in one launch (paged_decode_attention_append), with --separate as the
two calls of the reference.
Default workload: benchmark configuration 3 (Qwen3-8B shape, 32 q / 8 kv heads, D 128,
bf16, block 256, batch 64, context U[2048, 8192], 8192-block pool), synthetic
N(0,1) data resident in HBM, steps rotating over distinct layers of the
[2, layers, NB, 256, 8, 128] buffer so that no step re-reads what the previous
one left in the 256 MB MALL.

With --prefill the step is instead one paged prefill attention call (causal,
masks aligned bottom-right) over prompts whose K/V are already in the cache, at
the Qwen3-8B head shape; its roofline is the matrix cores (bf16 dense peak).

Prints ONE JSON line.  value = algorithmic bytes of (append + attention) per
step / wall time per step.  The attention call (pass-1 kernel + LSE merge
kernel) is also timed with HIP events on the stream it runs on: two events
bracketing the timed steps (one call per step in the default fused mode) ->
attn_us and roofline.  Where sequences share cache blocks (configuration 4's
prefix) the call is the cascaded entry and the algorithmic bytes count each
distinct cache row once; the per-sequence count is reported beside them.
The step's K/V/q bytes come from a seeded host generator and are uploaded, so
cpu_baseline -- the C oracle (test infrastructure, reference semantics) over
the whole step on the same bytes -- also checks the GPU step's output
(parity_vs_cpu).  "configs" holds every benchmark configuration's fused call measured
in the same run (device-generated N(0,1) data).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "vllm-oxide_amd"))
sys.path.insert(0, str(REPO))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, published
# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE summary of the same workload (calibrated HBM
# bytes per attention call); the committed summary names the config it covers.
TRAFFIC_PROFILE = {(2, False): REPO / "profiles" / "paged_decode_cfg2.md",
                   (3, False): REPO / "profiles" / "paged_decode_cfg3.md",
                   (4, False): REPO / "profiles" / "paged_decode_cfg4.md",
                   (5, False): REPO / "profiles" / "paged_decode_cfg5.md"}


def _profile_value(path, key: str):
    if path is None or not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith(key + ":"):
            return int(line.split(":")[1])
    return None


# Decode pass 1 as reported by split_tokens(): > 0 split grid, 0 persistent, -1 stream, -2 rows.
PASS1_NAMES = {"split": "split grid", "persistent": "persistent balanced", "stream": "wave-level stream",
               "rows": "whole-row stream"}
PASS1_KERNELS = {"split": "paged_decode_split + paged_decode_merge",
                 "persistent": "paged_decode_persistent + paged_decode_merge_persistent",
                 "stream": "paged_decode_stream + paged_decode_merge_stream",
                 "rows": "paged_decode_rows + paged_decode_merge_stream"}


def _pass1(split_tokens: int) -> str:
    return ("split" if split_tokens > 0 else "persistent" if split_tokens == 0 else
            "stream" if split_tokens == -1 else "rows")


def profiled_traffic(config: int, separate: bool):
    return _profile_value(TRAFFIC_PROFILE.get((config, separate)), "traffic_bytes_per_attention_call")


# PMC traffic of the prologue at its default size (16,384 tokens, Qwen3-8B heads).
PROLOGUE_PROFILE = REPO / "profiles" / "qk_norm_rope_cache_16k.md"


def host_workload(st, seed: int):
    """The decode step's inputs as host bytes, from the library's seeded generator: K and
    V of the blocks the batch uses (block ids renumbered 0 .. n-1 in first-use order),
    q, and the new token's K/V.  The GPU run uploads these exact bytes and the CPU
    baseline computes on them."""
    import numpy as np

    from oxide_paged_kv.workload import fill_normal

    c = st.cfg
    used = list(dict.fromkeys([int(x) for r in st.block_rows for x in r] + [int(x) for x in st.cow_pairs[:, 0]]))
    remap = {b: i for i, b in enumerate(used)}
    table = np.zeros_like(st.block_table)
    for b, r in enumerate(st.block_rows):
        table[b, :len(r)] = [remap[int(x)] for x in r]
    BS = c.block_size
    slots = np.array([remap[int(s) // BS] * BS + int(s) % BS for s in st.slot_mapping], np.int64)
    shape = (len(used), BS, c.num_kv_heads, c.head_dim)
    h = {"used": np.array(used, np.int64), "table": table, "slots": slots,
         "k": fill_normal(shape, seed, 1), "v": fill_normal(shape, seed, 2),
         "q": fill_normal((c.batch, c.num_heads, c.head_dim), seed, 3),
         "knew": fill_normal((c.batch, c.num_kv_heads, c.head_dim), seed, 4),
         "vnew": fill_normal((c.batch, c.num_kv_heads, c.head_dim), seed, 5)}
    if len(st.cow_pairs):  # copy-on-write before the append (the GPU side runs copy_blocks)
        for src, dst in st.cow_pairs:
            h["k"][remap[int(dst)]] = h["k"][remap[int(src)]]
            h["v"][remap[int(dst)]] = h["v"][remap[int(src)]]
    return h


def cpu_baseline(st, h, threads: int, min_seconds: float = 10.0):
    """The oracle's append + fp32-accumulated attention over the WHOLE step (every
    sequence of the batch), on the same bytes the GPU run uses; repeated until
    min_seconds have passed (at least once).  Returns the baseline entry and the
    output of the last repetition (for the parity check of the bench workload).  The
    append writes h's K/V in place (the same rows every repetition)."""
    import oracle

    c = st.cfg
    k, v = h["k"], h["v"]
    scale = 1 / math.sqrt(c.head_dim)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.reshape_and_cache(h["knew"], h["vnew"], k, v, h["slots"])
        out = oracle.paged_decode_attention(h["q"], k, v, st.cu_seqlens_k, h["table"], scale, c.window_left,
                                            "bf16", threads=threads)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            break
    step_bytes = st.attn_bytes() + st.append_bytes()
    entry = {"value": round(step_bytes * reps / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
             "host_nproc": os.cpu_count(), "kind": "port",
             "sample": f"the whole step: all {c.batch} sequences ({int(st.context_lens.sum())} keys), append + "
                       f"fp32-accumulated attention (C oracle, {threads} threads) on the bytes the GPU run "
                       f"uploads, {reps} reps in {dt:.1f} s"}
    return entry, out


def parity_vs_cpu(got, want) -> dict:
    """Bench-workload parity: the GPU step's output against the CPU baseline's, with the
    target's tolerance (max-abs 2e-2, max-rel 1e-2 floored at 1) and the error bar
    scaled to each (sequence, head) row (2e-2 max|row| + 1 bf16 ulp)."""
    import numpy as np

    got = got.astype(np.float64).reshape(-1, got.shape[-1])
    want = want.astype(np.float64).reshape(-1, want.shape[-1])
    err = np.abs(got - want)
    mag = np.abs(want).max(axis=1)
    ulp = np.exp2(np.floor(np.log2(np.maximum(mag, 2.0 ** -126))) - 7)
    row_ok = err.max(axis=1) <= 2e-2 * mag + ulp
    max_abs = float(err.max())
    max_rel = float((err / np.maximum(np.abs(want), 1.0)).max())
    return {"max_abs": round(max_abs, 6), "max_rel": round(max_rel, 6),
            "max_err_over_row_max": round(float((err.max(axis=1) / np.maximum(mag, 1e-30)).max()), 6),
            "ok": bool(np.isfinite(got).all() and max_abs <= 2e-2 and max_rel <= 1e-2 and row_ok.all())}


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16, published


def prefill_flops(lq: int, lk: int, heads: int, head_dim: int, window: int = -1) -> int:
    """QK^T + PV flops of one sequence over the keys each query sees (masked keys excluded)."""
    keys = 0
    for i in range(lq):
        hi = i + lk - lq
        lo = 0 if window < 0 else max(0, hi - window)
        keys += max(0, hi - lo + 1) if hi >= 0 else 0
    return 4 * head_dim * heads * keys


def prefill_cpu_baseline(seed: int, threads: int, min_seconds: float = 10.0) -> dict:
    """Oracle prefill attention on one 512-token prompt of the same head shape."""
    import numpy as np

    import oracle

    rng = np.random.default_rng(seed)
    L, Hq, Hkv, D, BS = 512, 32, 8, 128, 256

    def bits(shape):
        return oracle.f32_to_bf16_bits(rng.standard_normal(size=shape, dtype=np.float32)).reshape(shape)

    nb = L // BS
    kc, vc, q = bits((nb, BS, Hkv, D)), bits((nb, BS, Hkv, D)), bits((L, Hq, D))
    table = np.arange(nb, dtype=np.int32)[None]
    cu = np.array([0, L], np.uint32)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.prefill_attention(q, kc, vc, cu, cu, 1 / math.sqrt(D), table, -1, "bf16", threads=threads)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            break
    flops = prefill_flops(L, L, Hq, D)
    return {"value": round(flops * reps / dt / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"one {L}-token prompt, Qwen3-8B heads, fp32-accumulated, {reps} reps in {dt:.1f} s"}


def measure_prefill(dev, B: int, Lq: int, P: int, seed: int, steps: int, warmup: int) -> dict:
    """One paged prefill attention call (B prompts of Lq new tokens behind P cached tokens,
    Qwen3-8B heads) timed with two HIP events bracketing `steps` calls on the launch
    stream, the calls alternating between two layers' caches."""
    import torch

    import oxide_paged_kv as ox

    Lk = Lq + P
    Hq, Hkv, D, BS = 32, 8, 128, 256
    nb = (Lk + BS - 1) // BS
    g = torch.Generator(device=dev).manual_seed(seed)
    layers = 2
    kc = torch.randn((layers, B * nb, BS, Hkv, D), generator=g, device=dev).bfloat16()
    vc = torch.randn((layers, B * nb, BS, Hkv, D), generator=g, device=dev).bfloat16()
    q = torch.randn((layers, B * Lq, Hq, D), generator=g, device=dev).bfloat16()
    perm = torch.randperm(B * nb, generator=torch.Generator().manual_seed(seed)).int()
    table = perm.view(B, nb).to(dev)
    cuq = (torch.arange(B + 1, dtype=torch.int32) * Lq).to(dev)
    cuk = (torch.arange(B + 1, dtype=torch.int32) * Lk).to(dev)
    out = torch.empty((B * Lq, Hq, D), dtype=torch.bfloat16, device=dev)
    scale = 1 / math.sqrt(D)

    def call(i):
        ox.prefill_attn(q[i % layers], kc[i % layers], vc[i % layers], cuq, cuk, Lq, Lk, scale, table,
                        None, out)

    for i in range(warmup):
        call(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        call(i)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    us = e0.elapsed_time(e1) / steps * 1e3
    flops = B * prefill_flops(Lq, Lk, Hq, D)
    tflops = flops / (us * 1e-6) / 1e12
    del kc, vc, q, out
    torch.cuda.empty_cache()
    return {"workload": f"prefill-qwen3-8b-{B}x{Lq}" + (f"-prefix{P}" if P else ""),
            "prompts": B, "prompt_len": Lq, "prefix": P, "num_heads": Hq, "num_kv_heads": Hkv,
            "head_dim": D, "block_size": BS, "kernel": "paged_prefill_attn", "calls": steps,
            "call_us": round(us, 2), "wall_ms_per_call": round(wall * 1e3 / steps, 4),
            "tflops": round(tflops, 2), "algorithmic_flops": flops,
            "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "peak_tflops": MFMA_BF16_PEAK_TFLOPS}


def prefill_main(args) -> int:
    import torch

    dev = torch.device("cuda:0")
    m = measure_prefill(dev, args.prompts, args.prompt_len, args.prefix, args.seed, args.steps, args.warmup)
    res = {
        "metric": "paged prefill attention TFLOP/s (causal, Qwen3-8B heads)",
        "value": m["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": m["wall_ms_per_call"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) Q/K/V, seeded random block tables",
        "config": {k: m[k] for k in ("workload", "prompts", "prompt_len", "prefix", "num_heads", "num_kv_heads",
                                     "head_dim", "block_size")},
        "call_us": m["call_us"],
        "roofline": {"bound": "mfma", "achieved": m["tflops"], "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": m["frac"], "traffic": None,
                     "kernel": "paged_prefill_attn", "algorithmic_flops": m["algorithmic_flops"]},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = prefill_cpu_baseline(args.seed, min(16, os.cpu_count() or 1))
    print(json.dumps(res), flush=True)
    return 0


def prologue_bytes(tokens: int, hq: int, hkv: int, d: int) -> int:
    """HBM bytes of one qk_norm_rope_and_cache call: the qkv rows read, q written, k and v
    written to their slots, one fp32 cos/sin row, the position and the slot per token
    (the [D] norm weights stay in cache)."""
    return tokens * ((hq + 2 * hkv) * d * 2 + hq * d * 2 + 2 * hkv * d * 2 + d * 4 + 4 + 8)


def prologue_cpu_baseline(seed: int, min_seconds: float = 10.0) -> dict:
    import numpy as np

    import oracle

    rng = np.random.default_rng(seed)
    T, Hq, Hkv, D = 256, 32, 8, 128
    qkv = oracle.f32_to_bf16_bits(rng.standard_normal(size=(T, (Hq + 2 * Hkv) * D), dtype=np.float32))
    w = oracle.f32_to_bf16_bits(np.ones(D, np.float32))
    cs = oracle.rope_cos_sin_cache(8192, D, 1_000_000.0)
    pos = rng.integers(0, 8192, T).astype(np.int32)
    kc = np.zeros((T, Hkv, D), np.uint16)
    vc = np.zeros_like(kc)
    slots = np.arange(T, dtype=np.int64)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.qk_norm_rope_and_cache(qkv, Hq, Hkv, D, w, w, 1e-6, cs, pos, kc, vc, slots)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            break
    return {"value": round(prologue_bytes(T, Hq, Hkv, D) * reps / dt / 1e9, 4), "unit": "GB/s", "cores": 1,
            "kind": "port", "sample": f"{T} tokens, Qwen3-8B heads, scalar C, {reps} reps in {dt:.1f} s"}


def measure_prologue(dev, T: int, seed: int, steps: int, warmup: int) -> dict:
    """One qk_norm_rope_and_cache call over T tokens (Qwen3-8B heads) timed with two HIP
    events bracketing `steps` calls on the launch stream, the calls rotating over four
    layers' qkv rows."""
    import torch

    import oxide_paged_kv as ox

    Hq, Hkv, D, BS = 32, 8, 128, 256
    layers = 4
    g = torch.Generator(device=dev).manual_seed(seed)
    qkv = torch.randn((layers, T, (Hq + 2 * Hkv) * D), generator=g, device=dev).bfloat16()
    w = (1 + 0.1 * torch.randn((2, D), generator=g, device=dev)).bfloat16()
    cs = ox.rope_cos_sin_cache(32768, D, 1_000_000.0, dev)
    # Prefill-sized calls: prompts of 4096 tokens at positions 0..4095; decode-sized
    # calls (<= 256 tokens, one per sequence): scattered positions.
    if T > 256:
        pos = (torch.arange(T, device=dev, dtype=torch.int32) % 4096).contiguous()
    else:
        pos = torch.randint(0, 32768, (T,), generator=g, device=dev, dtype=torch.int32)
    nb = (T + BS - 1) // BS
    kc = torch.zeros((nb, BS, Hkv, D), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    slots = torch.randperm(nb * BS, generator=g, device=dev)[:T].contiguous()

    q_out = torch.empty((T, Hq, D), dtype=torch.bfloat16, device=dev)
    layer_qkv = [qkv[i] for i in range(layers)]

    def call(i):
        ox.qk_norm_rope_and_cache(layer_qkv[i % layers], Hq, Hkv, w[0], w[1], 1e-6, cs, pos, kc, vc, slots,
                                  q_out=q_out)

    for i in range(warmup):
        call(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        call(i)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    us = e0.elapsed_time(e1) / steps * 1e3
    nbytes = prologue_bytes(T, Hq, Hkv, D)
    gbps = nbytes / (us * 1e-6) / 1e9
    del qkv, kc, vc, q_out
    torch.cuda.empty_cache()
    return {"workload": f"prologue-qwen3-8b-{T}tok", "tokens": T, "num_heads": Hq, "num_kv_heads": Hkv,
            "head_dim": D, "kernel": "qk_norm_rope_cache_kernel", "calls": steps, "call_us": round(us, 2),
            "wall_ms_per_call": round(wall * 1e3 / steps, 4), "gbps": round(gbps, 1),
            "algorithmic_bytes": nbytes, "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": _profile_value(PROLOGUE_PROFILE, "traffic_bytes_per_call") if T == 16384 else None}


def prologue_main(args) -> int:
    import torch

    dev = torch.device("cuda:0")
    m = measure_prologue(dev, args.tokens, args.seed, args.steps, args.warmup)
    res = {
        "metric": "fused q/k RMSNorm + RoPE + KV append GB/s (Qwen3-8B heads)",
        "value": m["gbps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": m["wall_ms_per_call"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic N(0,1) qkv rows, random slots; positions 0..4095 per prompt (T > 256) or random",
        "config": {k: m[k] for k in ("workload", "tokens", "num_heads", "num_kv_heads", "head_dim")},
        "call_us": m["call_us"],
        "roofline": {"bound": "hbm", "achieved": m["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": m["frac"], "traffic": m["traffic"],
                     "kernel": "qk_norm_rope_cache_kernel", "algorithmic_bytes": m["algorithmic_bytes"]},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = prologue_cpu_baseline(args.seed)
    print(json.dumps(res), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 200; --prologue 500)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (default 100; --prologue 300)")
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--layers", type=int, default=0, help="distinct layers to rotate over (0 = auto)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--path", choices=["auto", "split", "persistent", "stream", "rows"], default="auto",
                    help="decode pass 1 (default: the library's choice by shape)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-config measurements of the other benchmark configurations")
    ap.add_argument("--separate", action="store_true",
                    help="append and attention as two calls (default: one fused call)")
    ap.add_argument("--prefill", action="store_true",
                    help="time paged prefill attention instead of the decode step")
    ap.add_argument("--prompts", type=int, default=4, help="--prefill: prompts per call")
    ap.add_argument("--prompt-len", type=int, default=4096, help="--prefill: new tokens per prompt")
    ap.add_argument("--prefix", type=int, default=0, help="--prefill: cached tokens before each prompt")
    ap.add_argument("--prologue", action="store_true",
                    help="time the fused q/k norm + RoPE + KV append instead of the decode step")
    ap.add_argument("--tokens", type=int, default=16384, help="--prologue: tokens per call")
    args = ap.parse_args()
    # A prologue call is ~0.1 ms: more of them keep the timed region near 50 ms.
    if args.steps is None:
        args.steps = 500 if args.prologue else 200
    if args.warmup is None:
        # The prologue's first ~200 calls run slower while the clocks ramp.
        args.warmup = 300 if args.prologue else 100
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        return 2
    if args.prefill:
        return prefill_main(args)
    if args.prologue:
        return prologue_main(args)

    return decode_main(args)


def _device_step_inputs(st, layers: int, dev, seed: int):
    """Per-config timing inputs generated on the GPU (N(0,1), seeded): the cache buffer
    [2, layers, NB, BS, Hkv, D] and per-layer q / new K / new V."""
    import numpy as np
    import torch

    c = st.cfg
    g = torch.Generator(device=dev).manual_seed(seed)
    buf = torch.empty((2, layers, st.pool_blocks, c.block_size, c.num_kv_heads, c.head_dim), dtype=torch.bfloat16,
                      device=dev)
    for kv in range(2):
        for layer in range(layers):
            buf[kv, layer].normal_(generator=g)
    q = torch.randn((layers, c.batch, c.num_heads, c.head_dim), generator=g, device=dev).bfloat16()
    knew = torch.randn((layers, c.batch, c.num_kv_heads, c.head_dim), generator=g, device=dev).bfloat16()
    vnew = torch.randn((layers, c.batch, c.num_kv_heads, c.head_dim), generator=g, device=dev).bfloat16()
    meta = (torch.from_numpy(st.slot_mapping).to(dev), torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(dev),
            torch.from_numpy(st.block_table).to(dev))
    return buf, q, knew, vnew, meta


def measure_config(cfg_id: int, dev, seed: int, steps: int = 100, warmup: int = 50) -> dict:
    """One benchmark configuration's fused append + attention call, averaged over `steps` calls
    bracketed by two HIP events on the launch stream (no events between calls), the
    steps rotating over the config's layers (cfg2: its 28 layers; others 4 layers, so no
    call re-reads what the previous one left in the 256 MB MALL)."""
    import torch

    import oxide_paged_kv as ox
    from oxide_paged_kv.workload import CONFIGS, make_decode_step

    cfg = CONFIGS[cfg_id]
    st = make_decode_step(cfg, seed=seed)
    layers = cfg.layers if cfg.layers > 1 else 4
    buf, q, knew, vnew, (sm, cu, bt) = _device_step_inputs(st, layers, dev, seed)
    out = torch.empty((cfg.batch, cfg.num_heads, cfg.head_dim), dtype=torch.bfloat16, device=dev)
    ws = torch.empty(max(ox.workspace_size(cfg.batch, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim,
                                           st.max_seqlen_k), 1), dtype=torch.uint8, device=dev)
    scale = 1 / math.sqrt(cfg.head_dim)
    window = None if cfg.window_left < 0 else cfg.window_left
    res = {}
    if len(st.cow_pairs):
        # Copy-on-write of the shared partial block, once per sequence, before the append.
        pairs = torch.from_numpy(st.cow_pairs).to(dev)
        ox.copy_blocks(buf[0, 0], buf[1, 0], pairs)
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record()
        for layer in range(layers):
            ox.copy_blocks(buf[0, layer], buf[1, layer], pairs)
        c1.record()
        torch.cuda.synchronize()
        cow_us = c0.elapsed_time(c1) / layers * 1e3
        cow_bytes = len(st.cow_pairs) * 2 * 2 * (cfg.block_size * cfg.num_kv_heads * cfg.head_dim * 2) + \
            16 * len(st.cow_pairs)
        res["cow_copy_blocks_us"] = round(cow_us, 2)
        res["cow_copy_blocks_gbps"] = round(cow_bytes / (cow_us * 1e-6) / 1e9, 1)

    # A batch whose block tables share a prefix (cfg4) runs the cascaded entry: the
    # shared blocks attended once for all sequences (the hint is an upper bound; the
    # library finds the shared count on the device).  The plain call is timed too.
    hint = cfg.shared_prefix // cfg.block_size if cfg.shared_prefix else None
    if hint:
        ws = torch.empty(ox.shared_prefix_workspace_size(cfg.batch, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim,
                                                         cfg.block_size, st.max_seqlen_k, hint),
                         dtype=torch.uint8, device=dev)

    def call(i, cascade=True):
        layer = i % layers
        ox.decode_attn(q[layer], buf[0, layer], buf[1, layer], cu, bt, st.max_seqlen_k, scale, window,
                       cfg.block_size, out=out, workspace=ws, append=(knew[layer], vnew[layer], sm),
                       shared_prefix_blocks=hint if cascade else None)

    def timed(cascade=True):
        for i in range(warmup):
            call(i, cascade)
        torch.cuda.synchronize()
        # A few ms of device work ahead of the bracket (a fill of a 4 GiB buffer, twice), so
        # the host has enqueued the timed calls before the GPU reaches them: for calls shorter
        # than their Python launch cost (cfg1) the bracket then times the device, not the host.
        filler = torch.empty(1 << 31, dtype=torch.int16, device=dev)
        filler.fill_(1)
        filler.fill_(2)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            call(warmup + i, cascade)
        e1.record()
        torch.cuda.synchronize()
        del filler
        return e0.elapsed_time(e1) / steps * 1e3

    if hint:
        plain_us = timed(cascade=False)
        res["no_cascade_attn_us"] = round(plain_us, 2)
    us = timed()
    # With shared blocks the algorithmic bytes count each distinct cache row once (the
    # least a call that reads a shared row once must move); the bytes a per-sequence
    # read would move (the reference's) are reported beside them.
    ref_bytes = st.attn_bytes() + st.append_bytes()
    nbytes = st.attn_unique_bytes() + st.append_bytes()
    gbps = nbytes / (us * 1e-6) / 1e9
    split = ox.split_tokens(cfg.batch, cfg.num_kv_heads, st.max_seqlen_k, num_heads=cfg.num_heads,
                            head_dim=cfg.head_dim, page_block_size=cfg.block_size)
    traffic = profiled_traffic(cfg_id, False)
    pass1 = PASS1_NAMES[_pass1(split)] if not hint else \
        "cascade: shared-prefix pass (paged_prefill_attn prefix mode) + wave-level stream over the rest"
    res.update({"workload": cfg.name, "pass1": pass1, "attn_us": round(us, 2),
                "algorithmic_bytes": nbytes, "attn_gbps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4),
                "traffic": traffic, "tokens_per_s": round(cfg.batch / (us * 1e-6), 1),
                "calls": steps, "layers_rotated": layers})
    if traffic:
        # HBM bytes the call actually moves (rocprofv3 FETCH_SIZE + WRITE_SIZE summary
        # under profiles/) over the same time.
        res["hbm_frac"] = round(traffic / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)
    if ref_bytes != nbytes:
        res["reference_equivalent_bytes"] = ref_bytes
        res["reference_equivalent_gbps"] = round(ref_bytes / (us * 1e-6) / 1e9, 1)
    if cfg.layers > 1:
        res["step_us_all_layers"] = round(us * cfg.layers, 1)
    del buf
    torch.cuda.empty_cache()
    return res


def decode_main(args) -> int:
    import numpy as np
    import torch

    import oxide_paged_kv as ox
    from oxide_paged_kv.workload import CONFIGS, make_decode_step

    cfg = CONFIGS[args.config]
    path = ox.DECODE_PATHS[args.path]
    dev = torch.device("cuda:0")
    st = make_decode_step(cfg, seed=args.seed)
    layers = args.layers or (cfg.layers if cfg.layers > 1 else 4)
    NB, BS, H, D = st.pool_blocks, cfg.block_size, cfg.num_kv_heads, cfg.head_dim
    # Host bytes of the step (also what the CPU baseline computes on), uploaded into
    # every rotated layer's blocks: each layer holds the same data at its own address.
    h = host_workload(st, args.seed)
    used = torch.from_numpy(h["used"]).to(dev)

    def up(a):
        return torch.from_numpy(a.view(np.int16)).to(dev).view(torch.bfloat16)

    # PagedKVCache buffer [2, L, NB, BS, H, D] (attention/mod.rs:55-85).
    buf = torch.zeros((2, layers, NB, BS, H, D), dtype=torch.bfloat16, device=dev)
    kd, vd = up(h["k"]), up(h["v"])
    for layer in range(layers):
        buf[0, layer].index_copy_(0, used, kd)
        buf[1, layer].index_copy_(0, used, vd)
    del kd, vd
    q, knew, vnew = up(h["q"]), up(h["knew"]), up(h["vnew"])
    # Metadata uploaded once per step for all layers (not once per layer).
    sm = torch.from_numpy(st.slot_mapping).to(dev)
    cu = torch.from_numpy(st.cu_seqlens_k.view(np.int32)).to(dev)
    bt = torch.from_numpy(st.block_table).to(dev)
    out = torch.empty((cfg.batch, cfg.num_heads, D), dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(max(ox.workspace_size(cfg.batch, cfg.num_heads, H, D, st.max_seqlen_k), 1),
                     dtype=torch.uint8, device=dev)
    scale = 1 / math.sqrt(D)
    window = None if cfg.window_left < 0 else cfg.window_left
    if len(st.cow_pairs):
        pairs = torch.from_numpy(st.cow_pairs).to(dev)
        for layer in range(layers):
            ox.copy_blocks(buf[0, layer], buf[1, layer], pairs)
    # A batch sharing a block-table prefix (cfg4) takes the cascaded entry in the fused mode.
    hint = cfg.shared_prefix // BS if cfg.shared_prefix and not args.separate and args.path == "auto" else None
    if hint:
        ws = torch.zeros(ox.shared_prefix_workspace_size(cfg.batch, cfg.num_heads, H, D, BS, st.max_seqlen_k, hint),
                         dtype=torch.uint8, device=dev)

    def step(i, ev=None):
        layer = i % layers
        kc, vc = buf[0, layer], buf[1, layer]
        if ev:
            ev[0].record()
        if args.separate:
            ox.reshape_and_cache(knew, vnew, kc, vc, sm)
            if ev:
                ev[1].record()
            ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale, window, BS, out=out, workspace=ws, path=path)
        else:
            if ev:
                ev[1].record()
            ox.decode_attn(q, kc, vc, cu, bt, st.max_seqlen_k, scale, window, BS, out=out,
                           workspace=ws, append=(knew, vnew, sm), path=path, shared_prefix_blocks=hint)
        if ev:
            ev[2].record()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # The timed steps carry no events (recording three per step costs about
    # 12 us of device time each on cfg3); the per-call durations for the
    # roofline come from a second pass of the same steps with events around
    # each attention launch.
    # Two HIP events bracket the timed region on the launch stream (nothing is
    # recorded between the steps): in the fused mode a step is exactly one
    # attention call, so the bracketed time over the steps is the call's average
    # duration, back to back.
    # The same few ms of device work ahead of the bracket as the per-config entries queue
    # (two fills of a 4 GiB buffer): the host has then enqueued the first timed calls
    # before the GPU reaches them, and the first calls after an idle GPU (which run
    # ~2 % slower) fall inside the fills, so the figure does not depend on --warmup.
    filler = torch.empty(1 << 31, dtype=torch.int16, device=dev)
    torch.cuda.synchronize()
    f0 = torch.cuda.Event(enable_timing=True)
    b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    f0.record()
    filler.fill_(1)
    filler.fill_(2)
    b0.record()
    for i in range(args.steps):
        step(args.warmup + i)
    b1.record()
    torch.cuda.synchronize()
    # Wall clock over the timed steps: host time from before the fills to the end of the
    # last step, less the fills' own device time (f0 -> b0).
    wall = time.perf_counter() - t0 - f0.elapsed_time(b0) * 1e-3
    bracket_us = b0.elapsed_time(b1) / args.steps * 1e3
    del filler
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(args.warmup + i, evs[i])
    torch.cuda.synchronize()
    gpu_out = out.float().cpu().numpy()  # the last step's output (every layer holds the same inputs)
    att_ms = [e[1].elapsed_time(e[2]) for e in evs]
    ms_per_step = wall * 1e3 / args.steps
    # Shared blocks (the cascade): each distinct cache row counts once, as in measure_config.
    attn_bytes, app_bytes = (st.attn_unique_bytes() if hint else st.attn_bytes()), st.append_bytes()
    kv_bytes = st.unique_kv_read_bytes() if hint else st.kv_read_bytes()
    # Fused: the bracketed average.  Separate (append + attention per step): the
    # attention call's own events from the second pass.
    attn_us = float(np.mean(att_ms)) * 1e3 if args.separate else bracket_us
    # The timed call's algorithmic bytes: attention, plus the append when fused into it.
    call_bytes = attn_bytes if args.separate else attn_bytes + app_bytes
    attn_gbps = call_bytes / (attn_us * 1e-6) / 1e9
    value = (attn_bytes + app_bytes) / (ms_per_step * 1e-3) / 1e9
    # The append kernel on its own (reshape_and_cache), for append GB/s.  A few
    # attention calls are queued first so the GPU is still busy while the host
    # enqueues the short appends: the events then time the device, not the launches.
    for i in range(8):
        ox.decode_attn(q, buf[0, i % layers], buf[1, i % layers], cu, bt, st.max_seqlen_k,
                       scale, window, BS, out=out, workspace=ws)
    a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a0.record()
    for i in range(20):
        layer = i % layers
        ox.reshape_and_cache(knew, vnew, buf[0, layer], buf[1, layer], sm)
    a1.record()
    torch.cuda.synchronize()
    app_us = a0.elapsed_time(a1) / 20 * 1e3
    app_gbps = app_bytes / (app_us * 1e-6) / 1e9
    del buf
    torch.cuda.empty_cache()

    extra = {}
    # Achievable-bandwidth calibration: copy_blocks over 1 MiB blocks (read+write).
    nblk = 2048
    cbuf = torch.empty((2, 2 * nblk, BS, H, D), dtype=torch.bfloat16, device=dev)
    pairs = torch.stack([torch.arange(nblk), torch.arange(nblk, 2 * nblk)], 1).to(dev)
    for _ in range(3):
        ox.copy_blocks(cbuf[0], cbuf[1], pairs)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        ox.copy_blocks(cbuf[0], cbuf[1], pairs)
    e1.record()
    torch.cuda.synchronize()
    cbytes = 2 * nblk * 2 * (BS * H * D * 2)
    extra["stream_copy_gbps"] = round(cbytes / (e0.elapsed_time(e1) / 10 * 1e-3) / 1e9, 1)
    # Prefix-hit gather (gather_blocks): 1024 blocks of K and V picked at random from the
    # same buffer into contiguous [n * BS, Hkv, D] outputs (read + write of each block).
    ng = 1024
    gids = torch.randperm(2 * nblk, generator=torch.Generator().manual_seed(args.seed))[:ng].int().to(dev)
    gk = torch.empty((ng * BS, H, D), dtype=torch.bfloat16, device=dev)
    gv = torch.empty_like(gk)
    for _ in range(3):
        ox.gather_blocks(cbuf[0], cbuf[1], gids, gk, gv)
    e0.record()
    for _ in range(10):
        ox.gather_blocks(cbuf[0], cbuf[1], gids, gk, gv)
    e1.record()
    torch.cuda.synchronize()
    gbytes = ng * 2 * 2 * (BS * H * D * 2) + 4 * ng
    extra["gather_blocks_gbps"] = round(gbytes / (e0.elapsed_time(e1) / 10 * 1e-3) / 1e9, 1)
    del gk, gv
    del cbuf
    torch.cuda.empty_cache()

    if not args.no_configs and args.path == "auto" and not args.separate:
        # Every benchmark configuration's fused call, measured in this same run.
        extra["configs"] = {f"cfg{i}": measure_config(i, dev, args.seed) for i in (1, 2, 3, 4, 5)}
        # The next-row kernels of the same layer, measured in the same run (no CPU baselines
        # here; `--prefill` / `--prologue` run them alone with theirs): paged prefill
        # attention at two prompt shapes (matrix-core roofline) and the fused q/k norm +
        # RoPE + KV append over 16k tokens (HBM roofline).
        # ~60 ms of warm-up calls each: the first calls of a run of these MFMA-bound kernels
        # run slower while the clocks ramp (measured, 20 timed calls: 4 x 4096 673 us after
        # 5 warm-up calls, 598 us after 50, 581 us after 100 with 200 timed; 16 x 1024 254 /
        # 227 / 205 us).
        extra["prefill"] = {m["workload"]: m for m in
                            (measure_prefill(dev, 4, 4096, 0, args.seed, 40, 100),
                             measure_prefill(dev, 16, 1024, 0, args.seed, 100, 300))}
        # 300 warm-up calls: the first ~200 calls of a run of these short kernels are ~12 %
        # slower (measured: 82 us for calls 20-220, then 72 us).
        extra["prologue"] = measure_prologue(dev, 16384, args.seed, 200, 300)
        if extra["prologue"]["traffic"]:
            extra["prologue"]["traffic_over_algorithmic"] = round(
                extra["prologue"]["traffic"] / extra["prologue"]["algorithmic_bytes"], 4)

    split = ox.split_tokens(cfg.batch, H, st.max_seqlen_k, path=path, num_heads=cfg.num_heads, head_dim=D,
                            page_block_size=BS)
    res = {
        "metric": "paged-decode attn KV-read GB/s (% HBM peak) + append GB/s, Qwen3-8B shape",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) K/V/Q from a seeded host generator (the same bytes feed the CPU baseline), "
                "seeded random block tables",
        "config": {"workload": cfg.name, "batch": cfg.batch, "num_heads": cfg.num_heads,
                   "num_kv_heads": H, "head_dim": D, "block_size": BS, "pool_blocks": NB,
                   "ctx": [cfg.ctx_lo, cfg.ctx_hi], "window_left": cfg.window_left,
                   "layers_rotated": layers, "split_tokens": split, "pass1": PASS1_NAMES[_pass1(split)],
                   "total_keys": int(st.context_lens.sum())},
        "step_mode": "separate append + attention" if args.separate else "fused append + attention (one launch)",
        "attn_us": round(attn_us, 2),
        "attn_us_timing": ("attention call events, second pass of the steps" if args.separate else
                           "two events bracketing the timed steps (one attention call per step)"),
        # Per-call events (three recorded per step in a second pass; their own
        # overhead lengthens each call by a few us).
        "attn_us_per_call_events_p10_p50_p90": [round(float(np.percentile(att_ms, q)) * 1e3, 2)
                                                for q in (10, 50, 90)],
        "attn_kv_read_gbps": round(kv_bytes / (attn_us * 1e-6) / 1e9, 1),
        "attn_gbps": round(attn_gbps, 1),
        "attn_hbm_frac": round(attn_gbps / HBM_PEAK_GBPS, 4),
        "append_us": round(app_us, 2),
        "append_gbps": round(app_gbps, 1),
        "tokens_per_s": round(cfg.batch / (ms_per_step * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(attn_gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(attn_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": profiled_traffic(args.config, args.separate) if args.path == "auto" else None,
                     "kernel": ("paged_prefill_attn (shared-prefix mode) + " if hint else "")
                               + PASS1_KERNELS[_pass1(split)]
                               + " (one attention call" + ("" if args.separate else ", append fused") + ")",
                     "algorithmic_bytes": call_bytes},
        **extra,
    }
    if hint:
        ref_bytes = st.attn_bytes() + (0 if args.separate else app_bytes)
        res["reference_equivalent_bytes"] = ref_bytes
        res["reference_equivalent_gbps"] = round(ref_bytes / (attn_us * 1e-6) / 1e9, 1)
    if not args.no_cpu_baseline:
        threads = min(16, os.cpu_count() or 1)
        res["cpu_baseline"], cpu_out = cpu_baseline(st, h, threads)
        res["parity_vs_cpu"] = parity_vs_cpu(gpu_out, cpu_out)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
