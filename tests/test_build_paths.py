"""The build row of the drop-in boundary: the static archive links into a C program
(through the Makefile path, no Python, no shared library), and the Rust FFI crate and
the Makefile declare and compile exactly what the headers and build.py do."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "vllm-oxide_amd"
CRATE = REPO / "rust" / "oxide-paged-kv-sys"


def _header_functions():
    """name -> argument count of every function include/*.h declares."""
    out = {}
    for h in sorted((REPO / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^[a-z_0-9 ]*?\**\s*([a-z_][a-z_0-9]*)\s*\(([^)]*)\);", text, flags=re.M | re.S):
            args = [a for a in " ".join(m.group(2).split()).split(",") if a.strip() not in ("", "void")]
            out[m.group(1)] = len(args)
    return out


def _rust_functions():
    text = (CRATE / "src" / "lib.rs").read_text()
    block = text[text.index('extern "C" {'):]
    out = {}
    for m in re.finditer(r"pub fn (\w+)\((.*?)\)", block, flags=re.S):
        out[m.group(1)] = len([a for a in m.group(2).split(",") if a.strip()])
    return out


def test_rust_ffi_declares_every_header_function():
    want = _header_functions()
    got = _rust_functions()
    assert set(got) == set(want)
    for name, n in want.items():
        assert got[name] == n, (name, got[name], n)
    # the reference's two symbols keep its Rust parameter types (kernels.rs:15-36)
    text = (CRATE / "src" / "lib.rs").read_text()
    assert "slot_mapping: *const c_long,\n        num_tokens: c_long," in text
    assert "block_mapping: *const c_long,\n        num_pairs: c_long,\n        block_stride: c_long," in text


def test_build_flags_agree():
    """build.rs and the Makefile compile with build.py's device flags for gfx950."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("oxide_build", PKG / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    rs = (CRATE / "build.rs").read_text()
    mk = (PKG / "Makefile").read_text()
    for flag in ("-O3", "-std=c++17", "-fPIC", "-packed-fp32-ops"):
        assert flag in mod.HIP_FLAGS
        assert f'"{flag}"' in rs or flag in rs
        assert flag in mk
    assert 'unwrap_or_else(|_| "gfx950".into())' in rs and "ARCH     ?= gfx950" in mk
    assert "CARGO_FEATURE_ROCM" in rs and "rustc-link-lib=static=oxide_paged_kv" in rs
    assert "rustc-link-lib=dylib=amdhip64" in rs


@pytest.mark.skipif(shutil.which("make") is None, reason="make is not installed")
def test_static_archive_links_into_c_program():
    r = subprocess.run(["make", "-s", "-C", str(PKG), "static-test"], capture_output=True, text=True,
                       timeout=900)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "static link: 0 failures" in r.stdout


def test_kernels_do_not_spill():
    """Every kernel of the last build (build.py keeps the compiler's resource report
    next to the objects) runs without register spills or scratch memory, and the
    decode and prefill passes keep the occupancy their designs rely on: a spill
    reload is a vector load whose wait also drains the tile loads in flight."""
    import json

    res_file = PKG / "_build" / "kernel_resources.json"
    if not res_file.exists():
        pytest.skip("no build in this tree (run __graft_entry__.build())")
    res = json.loads(res_file.read_text())
    assert res, "empty resource report"
    spilling = {k: (v.get("VGPRs Spill"), v.get("SGPRs Spill"), v.get("ScratchSize [bytes/lane]"))
                for k, v in res.items()
                if v.get("VGPRs Spill", 0) or v.get("ScratchSize [bytes/lane]", 0)}
    assert not spilling, spilling
    occ = {k: v.get("Occupancy [waves/SIMD]") for k, v in res.items()}
    stream = [o for k, o in occ.items() if "paged_decode_stream" in k]
    prefill = [o for k, o in occ.items() if "paged_prefill_attn" in k]
    assert stream and min(stream) >= 2, stream
    assert prefill and min(prefill) >= 2, prefill
