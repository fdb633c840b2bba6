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


def _c_type(decl: str) -> str:
    """C parameter declaration -> its type with the name dropped, e.g.
    'const int64_t * slot_mapping' -> 'const int64_t*'."""
    decl = " ".join(decl.replace("*", " * ").split())
    words = decl.split(" ")
    if len(words) > 1 and re.fullmatch(r"[A-Za-z_]\w*", words[-1]) and words[-1] not in (
            "int", "float", "double", "char", "void", "size_t") and not words[-1].endswith("_t"):
        words = words[:-1]
    return " ".join(words).replace(" *", "*")


def _header_functions():
    """name -> (return type, [parameter types]) of every function include/*.h declares."""
    out = {}
    for h in sorted((REPO / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^([a-z_0-9 ]*?\**)\s*([a-z_][a-z_0-9]*)\s*\(([^)]*)\);", text,
                             flags=re.M | re.S):
            args = [a for a in " ".join(m.group(3).split()).split(",") if a.strip() not in ("", "void")]
            out[m.group(2)] = (_c_type(m.group(1)), [_c_type(a) for a in args])
    return out


# Rust FFI types -> the C type each must bind to on the LP64 hosts this library targets
# (c_long is 64 bits there, as the reference's kernels.rs:15-36 relies on for int64_t).
_RUST_TO_C = {"c_void": "void", "c_int": "int", "c_long": "int64_t", "c_char": "char",
              "i32": "int32_t", "u32": "uint32_t", "i64": "int64_t", "u64": "uint64_t",
              "f32": "float", "f64": "double", "usize": "size_t", "HipStream": "void*"}


def _rust_c_type(t: str) -> str:
    """'*const c_void' -> 'const void*', '*mut i64' -> 'int64_t*', 'HipStream' -> 'void*'."""
    t = " ".join(t.split())
    m = re.fullmatch(r"\*(const|mut) (.+)", t)
    if m:
        inner = _rust_c_type(m.group(2))
        return ("const " if m.group(1) == "const" else "") + inner + "*"
    if t not in _RUST_TO_C:
        raise AssertionError(f"unmapped Rust FFI type {t!r}")
    return _RUST_TO_C[t]


def _rust_functions():
    """name -> (return type, [parameter types]) of the crate's extern "C" block, in C terms."""
    text = (CRATE / "src" / "lib.rs").read_text()
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    block = re.sub(r"//[^\n]*", "", block)
    out = {}
    for m in re.finditer(r"pub fn (\w+)\((.*?)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        params = [a.split(":", 1)[1] for a in m.group(2).split(",") if a.strip()]
        ret = _rust_c_type(m.group(3).strip()) if m.group(3) else "void"
        out[m.group(1)] = (ret, [_rust_c_type(p) for p in params])
    return out


def _mismatches(want: dict, got: dict) -> list:
    bad = [("missing in Rust", n) for n in sorted(set(want) - set(got))]
    bad += [("not in the headers", n) for n in sorted(set(got) - set(want))]
    for name in sorted(set(want) & set(got)):
        (wr, wa), (gr, ga) = want[name], got[name]
        if wr != gr:
            bad.append((name, "return", gr, wr))
        if len(wa) != len(ga):
            bad.append((name, "arity", len(ga), len(wa)))
        bad += [(name, i, g, w) for i, (g, w) in enumerate(zip(ga, wa)) if g != w]
    return bad


def test_rust_ffi_declares_every_header_function():
    """Every function of include/*.h is declared in the Rust extern block with the same
    return type and the same parameter types, position by position (what a C compiler
    would check of the binding; no Rust toolchain in this image)."""
    want = _header_functions()
    got = _rust_functions()
    assert len(want) >= 19, sorted(want)
    assert not _mismatches(want, got), _mismatches(want, got)
    # the reference's two symbols keep its Rust parameter types (kernels.rs:15-36)
    text = (CRATE / "src" / "lib.rs").read_text()
    assert "slot_mapping: *const c_long,\n        num_tokens: c_long," in text
    assert "block_mapping: *const c_long,\n        num_pairs: c_long,\n        block_stride: c_long," in text


@pytest.mark.parametrize("swap", [("*const u32", "*const i32"), ("*const i32", "*const u32"),
                                  ("*const c_void", "*mut c_void"), ("usize", "c_long"), ("f32", "i32")])
def test_rust_ffi_type_check_catches_a_swap(swap, monkeypatch):
    """A scratch copy of the binding with one parameter type swapped fails the check."""
    text = (CRATE / "src" / "lib.rs").read_text()
    i = text.index('extern "C" {')
    a, b = swap
    j = text.index(": " + a + ",", i)
    bad = text[:j] + ": " + b + "," + text[j + len(a) + 3:]
    monkeypatch.setattr(Path, "read_text", lambda self, *args, **kw: bad)
    got = _rust_functions()
    monkeypatch.undo()
    assert _mismatches(_header_functions(), got)


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
    reload is a vector load whose wait also drains the tile loads in flight.
    SGPR spills are not memory spills on gfx950: the compiler parks those scalars in
    lanes of a VGPR (v_writelane / v_readlane, no memory access), and any that went to
    memory would show as scratch use, which is checked."""
    import json

    import importlib.util

    res_file = PKG / "_build" / "kernel_resources.json"
    if not res_file.exists():
        # A fresh tree: build it (the report is written by the build), so the check runs.
        spec = importlib.util.spec_from_file_location("oxide_build", PKG / "build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
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
