"""Shared helpers for the parity tests: seeded 16-bit data and torch <-> numpy bits."""
from __future__ import annotations

import numpy as np

import oracle


def normal_bits(rng: np.random.Generator, shape, dtype: str = "bf16", scale: float = 1.0) -> np.ndarray:
    """N(0, scale^2) values rounded (RNE) to bf16/f16, as uint16 bit patterns."""
    x = (rng.standard_normal(size=shape, dtype=np.float32) * np.float32(scale))
    if dtype == "bf16":
        return oracle.f32_to_bf16_bits(x).reshape(shape)
    return x.astype(np.float16).view(np.uint16).reshape(shape)


def to_torch(bits: np.ndarray, dtype: str, device):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device)
    return t.view(torch.bfloat16 if dtype == "bf16" else torch.float16)


def to_bits(t) -> np.ndarray:
    import torch

    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def to_f32(t) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_attn_close(got: np.ndarray, want: np.ndarray, atol: float = 2e-2, rtol: float = 1e-2):
    """Attention tolerance stated by the target: max-abs 2e-2 and max-rel 1e-2 (bf16
    output vs the fp32-accumulated oracle).  max-rel is taken as |got-want| /
    max(|want|, 1): relative to the value, floored at the unit scale of N(0,1)
    data so that near-zero outputs are judged by the absolute bound."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert np.all(np.isfinite(got)), "non-finite output"
    err = np.abs(got - want)
    max_abs = float(err.max()) if err.size else 0.0
    max_rel = float((err / np.maximum(np.abs(want), 1.0)).max()) if err.size else 0.0
    assert max_abs <= atol, f"max-abs {max_abs:.3e} > {atol}"
    assert max_rel <= rtol, f"max-rel {max_rel:.3e} > {rtol}"
    return max_abs, max_rel
