"""CPU checks of the C-ABI library: it loads, exports every symbol include/*.h
declares, and its host-side argument validation reports the documented errors
(no kernel is launched on these paths)."""
import re
from pathlib import Path

import ctypes
import pytest

REPO = Path(__file__).resolve().parent.parent


def _declared_functions():
    names = []
    for h in sorted((REPO / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"^[a-z_0-9 ]*?\**\s*([a-z_][a-z_0-9]*)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    import oxide_paged_kv
    from oxide_paged_kv import _lib

    L = oxide_paged_kv.load()
    declared = _declared_functions()
    assert {"reshape_and_cache", "copy_blocks", "gather_blocks", "paged_decode_attention"} <= set(declared)
    for name in declared:
        assert hasattr(L, name), f"{name} declared but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_error_paths_without_launch():
    from oxide_paged_kv import _lib

    L = _lib.load()
    L.oxide_clear_error()
    # Unknown dtype: the reference silently does nothing; here it is a recorded error.
    L.reshape_and_cache(None, None, None, None, None, 1, 8, 128, 7, None)
    assert L.oxide_last_error() == 2
    L.oxide_clear_error()
    # Empty batch: no-op, no error.
    L.reshape_and_cache(None, None, None, None, None, 0, 8, 128, 1, None)
    L.copy_blocks(None, None, None, 0, 1024, 1, None)
    L.gather_blocks(None, None, None, None, None, 0, 1024, 1, None)
    assert L.oxide_last_error() == 0
    L.copy_blocks(None, None, None, -1, 1024, 1, None)
    assert L.oxide_last_error() == 1
    L.oxide_clear_error()
    # Attention: unsupported head_dim / group size / dtype.
    args = [None] * 6 + [1, 1, 1]
    dummy = ctypes.c_void_p(16)
    ptrs = [dummy, dummy, dummy, dummy, dummy, dummy]
    L.paged_decode_attention(*ptrs, 1, 4, 1, 32, 8, 96, 256, 10, -1, 0.1, dummy, 1 << 30, 1, None)
    assert L.oxide_last_error() == 3
    L.oxide_clear_error()
    L.paged_decode_attention(*ptrs, 1, 4, 1, 72, 8, 128, 256, 10, -1, 0.1, dummy, 1 << 30, 1, None)  # group 9
    assert L.oxide_last_error() == 3
    L.oxide_clear_error()
    L.paged_decode_attention(*ptrs, 1, 4, 1, 32, 8, 128, 256, 10, -1, 0.1, dummy, 1 << 30, 2, None)
    assert L.oxide_last_error() == 2
    L.oxide_clear_error()
    L.paged_decode_attention(*ptrs, 1, 4, 1, 32, 8, 128, 256, 10, -1, 0.1, dummy, 0, 1, None)
    assert L.oxide_last_error() == 4
    L.oxide_clear_error()
    assert L.oxide_error_string(4) == b"workspace too small"
    del args


def test_workspace_and_split_policy():
    """Long shapes take the stream pass (-1), small ones a split grid; the workspace
    holds either path's partials (split: a row per (sequence, head, split); stream:
    two per (key range, kv head, query of the group), 8 ranges per CU per head set;
    without a GPU the CU count reads as 256)."""
    import oxide_paged_kv as ox

    assert ox.split_tokens(64, 8, 8192) == -1
    assert ox.split_tokens(32, 8, 4096) == 256
    assert ox.split_tokens(1, 1, 100) == 128
    ws = ox.workspace_size(64, 32, 8, 128, 8192)
    assert ws >= 2 * 256 * 8 * 4 * (128 + 1) * 4
    st = ox.split_tokens(64, 8, 8192, path="split")
    assert st % 256 == 0
    splits = -(-8192 // st)
    assert ox.workspace_size(64, 32, 8, 128, 8192) >= 64 * 32 * splits * (128 + 1) * 4
    # a forced path is an argument of that call only: the shape policy is unchanged after it
    assert ox.split_tokens(64, 8, 8192) == -1
    assert ox.workspace_size(64, 32, 8, 128, 0) == 0


def test_cascade_plan_and_workspace():
    """The cascaded entry's host policy (no launch): the plain entries where sharing
    saves under 200 MB of K/V reads, the cascade beyond, overlapped when the per-sequence
    part is long enough to hide the shared-key pass; shapes the stream pass does not take
    and a zero hint run the plain entries; the workspace covers both forms and the plain
    one.  Without a GPU the CU count reads as 256."""
    import oxide_paged_kv as ox

    plan = ox.shared_prefix_plan
    assert plan(4, 32, 8, 128, 256, 8192 + 256, 32) == "plain"        # 100 MB saved
    assert plan(64, 32, 8, 128, 256, 1024 + 3000, 4) == "overlap"     # 264 MB, long private parts
    assert plan(128, 32, 8, 128, 256, 4096 + 100, 16) == "serial"     # short private parts
    assert plan(128, 32, 8, 128, 256, 5120, 16) == "overlap"          # cfg4
    assert plan(128, 32, 8, 128, 256, 5120, 0) == "plain"
    assert plan(128, 36, 6, 128, 256, 5120, 16) == "plain"            # kv heads not dividing 8
    assert plan(128, 32, 8, 96, 256, 5120, 16) == "plain"             # head_dim not built
    ws = ox.shared_prefix_workspace_size(128, 32, 8, 128, 256, 5120, 16)
    assert ws >= ox.workspace_size(128, 32, 8, 128, 5120)
    # prefix partials: at least one split row per (sequence, head) plus the whole-sequence rows
    assert ws >= 2 * 128 * 32 * (128 + 1) * 4
    # a larger hint never needs less workspace; the hint is clamped to the longest sequence
    assert ox.shared_prefix_workspace_size(128, 32, 8, 128, 256, 5120, 8) <= ws
    assert ox.shared_prefix_workspace_size(128, 32, 8, 128, 256, 5120, 10 ** 6) == \
        ox.shared_prefix_workspace_size(128, 32, 8, 128, 256, 5120, 20)


def test_no_cpu_fallback_when_library_missing(tmp_path, monkeypatch):
    from oxide_paged_kv import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "missing.so")
    with pytest.raises(ImportError):
        _lib.load()
