"""Builds liboxide_paged_kv.so (gfx950 HIP kernels + C ABI + C++ host layer).

The library is built in-tree, next to this file, with plain hipcc calls (no
cmake, no JIT cache), so the .so travels with the source tree.  Every call
recompiles.  Counterpart of the reference's crates/vllm-oxide/build.rs:1-30
(nvcc via cudaforge -> static lib); here hipcc --offload-arch=gfx950 -> the
shared library Python loads with ctypes, plus the same objects archived as
liboxide_paged_kv.a.  rust/oxide-paged-kv-sys/build.rs and
vllm-oxide_amd/Makefile compile the same sources with the same flags.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
INCLUDE = REPO / "include"
BUILD = PKG / "_build"
LIB = PKG / "liboxide_paged_kv.so"
STATIC_LIB = PKG / "liboxide_paged_kv.a"
HOST_TEST_SRC = REPO / "tests" / "cpp" / "test_host.cpp"
HOST_TEST_BIN = REPO / "tests" / "cpp" / "build" / "test_host"
HOST_TEST_STAMP = HOST_TEST_BIN.with_suffix(".sources.sha256")
# Per-kernel register, scratch and LDS use reported by the compiler for the last build.
RESOURCES = BUILD / "kernel_resources.json"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in any kernel.
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp")) + sorted(HOST.glob("*.cpp"))


def _parse_resources(text: str) -> dict:
    """Kernel resource remarks (-Rpass-analysis=kernel-resource-usage) -> {kernel: {field: value}}."""
    import re

    out, cur = {}, None
    for line in text.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([A-Za-z][A-Za-z /\[\]]*?):\s+(\S+) \[-Rpass-analysis", line)
        if m and cur is not None:
            v = m.group(2)
            cur[m.group(1).strip()] = int(v) if v.lstrip("-").isdigit() else v
    return out


def _compile(src: Path):
    obj = BUILD / (src.parent.name + "_" + src.stem + ".o")
    cmd = [HIPCC, *HIP_FLAGS, "-I", str(INCLUDE), "-I", str(CSRC), "-I", str(HOST)]
    if src.suffix == ".cpp":
        cmd += ["-x", "hip"]
    else:
        cmd += ["-Rpass-analysis=kernel-resource-usage"]
    cmd += ["-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    return obj, _parse_resources(r.stderr)


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = _sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = list(ex.map(_compile, srcs))
    objs = [o for o, _ in results]
    import json

    resources = {}
    for _, res in results:
        resources.update(res)
    RESOURCES.write_text(json.dumps(resources, indent=1, sort_keys=True))
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(LIB), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    # The same objects as a static archive (what the Rust crate's build.rs and the
    # Makefile produce) for hosts that link the kernels statically.
    STATIC_LIB.unlink(missing_ok=True)
    r = subprocess.run(["ar", "rcs", str(STATIC_LIB), *map(str, objs)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"ar failed:\n{r.stdout}\n{r.stderr}")
    build_host_test()
    if verbose:
        print(f"built {LIB}")
    return LIB


def host_test_digest() -> str:
    """Digest of what the host test binary is built from: its source, the host layer,
    the header and the library it links (content, not mtimes, which a copied tree may
    not keep)."""
    import hashlib

    files = [HOST_TEST_SRC, INCLUDE / "oxide_paged_kv.h", LIB, *sorted(HOST.glob("*"))]
    h = hashlib.sha256()
    for f in files:
        h.update(f.name.encode())
        h.update(f.read_bytes() if f.exists() else b"<missing>")
    return h.hexdigest()


def host_test_current() -> bool:
    return HOST_TEST_BIN.exists() and HOST_TEST_STAMP.exists() and \
        HOST_TEST_STAMP.read_text().strip() == host_test_digest()


def build_host_test() -> Path:
    """C++ test binary of the host layer (tests/cpp/test_host.cpp), linked to the library;
    records the digest of its sources next to it."""
    HOST_TEST_BIN.parent.mkdir(parents=True, exist_ok=True)
    cmd = [HIPCC, *HIP_FLAGS, "-I", str(INCLUDE), "-I", str(HOST), "-I", str(PKG / "csrc"), str(HOST_TEST_SRC), "-o",
           str(HOST_TEST_BIN), "-L", str(PKG), "-loxide_paged_kv", f"-Wl,-rpath,{PKG}",
           "-Wl,-rpath,$ORIGIN/../../../vllm-oxide_amd"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {HOST_TEST_SRC.name}:\n{r.stdout}\n{r.stderr}")
    HOST_TEST_STAMP.write_text(host_test_digest())
    return HOST_TEST_BIN


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
