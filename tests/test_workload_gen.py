"""CPU checks of the host N(0, 1) generator that feeds the benchmark's GPU run and its
CPU baseline with the same bytes (oxide_fill_normal)."""
import numpy as np

import oracle


def test_fill_normal_deterministic_over_threads_and_streams():
    from oxide_paged_kv.workload import fill_normal

    a = fill_normal((1 << 20) + 3, seed=5, stream=1, threads=1)
    b = fill_normal((1 << 20) + 3, seed=5, stream=1, threads=7)
    assert np.array_equal(a, b)
    c = fill_normal((1 << 20) + 3, seed=5, stream=2, threads=7)
    d = fill_normal((1 << 20) + 3, seed=6, stream=1, threads=7)
    assert (a != c).mean() > 0.9 and (a != d).mean() > 0.9
    # a prefix of a longer fill is the shorter fill
    assert np.array_equal(fill_normal(1001, 5, 1), a[:1001])


def test_fill_normal_moments_and_rounding():
    from oxide_paged_kv.workload import fill_normal

    f = fill_normal(1 << 22, seed=0, stream=0, dtype="f32").astype(np.float64)
    assert abs(f.mean()) < 3e-3 and abs(f.var() - 1) < 5e-3
    # tails of a standard normal: P(|x| > 3) = 0.0027
    assert abs((np.abs(f) > 3).mean() - 0.0027) < 4e-4
    bf = fill_normal(1 << 22, seed=0, stream=0, dtype="bf16")
    assert np.array_equal(bf, oracle.f32_to_bf16_bits(f.astype(np.float32)))
    h = fill_normal(1 << 16, seed=0, stream=0, dtype="f16")
    assert np.array_equal(h, f[:1 << 16].astype(np.float32).astype(np.float16).view(np.uint16))
