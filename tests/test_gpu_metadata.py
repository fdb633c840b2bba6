"""GPU parity of build_decode_metadata_device against the oracle's host restatement
(compute_slot_mapping at position L-1 and build_decode_metadata), bit-exact."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _expected(lens, rows, bs):
    cu_q, cu_k, _ = oracle.build_decode_metadata(lens)
    slots = []
    for L, r in zip(lens, rows):
        slots.append(-1 if L == 0 else int(oracle.compute_slot_mapping(r, bs, int(L) - 1, 1)[0]))
    return cu_k, np.array(slots, np.int64)


@pytest.mark.parametrize("B,bs,seed", [(1, 256, 0), (64, 256, 1), (3000, 16, 2), (5, 32, 3)])
def test_device_metadata_matches_oracle(device, B, bs, seed):
    import torch
    import oxide_paged_kv as ox

    rng = np.random.default_rng(seed)
    lens = rng.integers(0, 8 * bs, size=B).astype(np.uint32)
    lens[::7] = 0
    rows = [rng.integers(0, 10 ** 6, size=(int(L) + bs - 1) // bs).astype(np.int32) for L in lens]
    table = oracle.pad_block_table(rows) if any(len(r) for r in rows) else np.zeros((B, 1), np.int32)
    cu, slots = ox.build_decode_metadata(torch.from_numpy(lens.view(np.int32)).to(device),
                                         torch.from_numpy(np.ascontiguousarray(table)).to(device), bs)
    want_cu, want_slots = _expected(lens, rows, bs)
    assert np.array_equal(cu.cpu().numpy().view(np.uint32), want_cu)
    assert np.array_equal(slots.cpu().numpy(), want_slots)


def test_device_metadata_reference_decode_vectors(device):
    """metadata.rs:94-103 (context lens 5, 20, 3 -> cu 0,5,25,28) with tables whose
    new-token slots follow kv_cache_manager.rs's formula."""
    import torch
    import oxide_paged_kv as ox

    lens = np.array([5, 20, 3], np.uint32)
    table = np.array([[7], [2], [9]], np.int32)
    cu, slots = ox.build_decode_metadata(torch.from_numpy(lens.view(np.int32)).to(device),
                                         torch.from_numpy(table).to(device), 256)
    assert cu.cpu().numpy().tolist() == [0, 5, 25, 28]
    assert slots.cpu().numpy().tolist() == [7 * 256 + 4, 2 * 256 + 19, 9 * 256 + 2]
