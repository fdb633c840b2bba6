"""Runs the C++ host-layer tests (tests/cpp/test_host.cpp).

CPU: block pool, slot mapping, metadata, padding and layout, restating the
reference's unit tests; XXH64 of the host layer against python-xxhash.
GPU: PagedKVCache append known answer, a DecodeStep against fp64 softmax, and a
DecodeStep over a shared-prefix batch (the cascaded entry) against the plain entry."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
BIN = REPO / "tests" / "cpp" / "build" / "test_host"


def _binary():
    """The host test binary, rebuilt when it is missing or was built from other sources
    (build.py keeps a digest of them next to it)."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("oxide_build", REPO / "vllm-oxide_amd" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    if not mod.host_test_current():
        mod.build_host_test()
    return BIN


def test_host_layer_cpu():
    r = subprocess.run([str(_binary()), "cpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "cpu: 0 failures" in r.stdout


def test_host_xxh64_matches_python_xxhash():
    import xxhash

    rng = np.random.default_rng(3)
    for n in [0, 3, 8, 31, 32, 33, 100, 1028]:
        data = rng.integers(0, 256, n).astype(np.uint8).tobytes()
        for seed in (0, 7):
            r = subprocess.run([str(_binary()), "hash", str(seed), data.hex() or "x"],
                               capture_output=True, text=True, timeout=60)
            assert r.returncode == 0
            assert int(r.stdout) == xxhash.xxh64_intdigest(data, seed=seed), (n, seed)


@pytest.mark.gpu
def test_host_layer_gpu(device):
    r = subprocess.run([str(_binary()), "gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "gpu: 0 failures" in r.stdout
