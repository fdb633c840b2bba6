// build.rs -- counterpart of crates/vllm-oxide/build.rs:1-30 (nvcc via cudaforge ->
// libvllmoxidekernels.a, links cudart, gated by CARGO_FEATURE_CUDA).  Here, gated by
// CARGO_FEATURE_ROCM: every HIP / C++ source of vllm-oxide_amd is compiled by hipcc
// for gfx950 with the flags of vllm-oxide_amd/build.py and its Makefile, archived into
// liboxide_paged_kv.a in OUT_DIR, and linked statically with amdhip64 and the C++
// runtime as dynamic dependencies.
//
// Environment: HIPCC (default /opt/rocm/bin/hipcc), OXIDE_OFFLOAD_ARCH (default gfx950),
// ROCM_PATH (default /opt/rocm) for the amdhip64 search path.
use std::env;
use std::path::{Path, PathBuf};
use std::process::{Child, Command};

fn sources(dir: &Path, ext: &str) -> Vec<PathBuf> {
    let mut v: Vec<PathBuf> = std::fs::read_dir(dir)
        .unwrap_or_else(|e| panic!("read {}: {e}", dir.display()))
        .filter_map(|e| e.ok().map(|e| e.path()))
        .filter(|p| p.extension().map_or(false, |x| x == ext))
        .collect();
    v.sort();
    v
}

fn main() {
    if env::var("CARGO_FEATURE_ROCM").is_err() {
        return;
    }
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let root = manifest.join("../..").canonicalize().expect("repository root");
    let pkg = root.join("vllm-oxide_amd");
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".into());
    let arch = env::var("OXIDE_OFFLOAD_ARCH").unwrap_or_else(|_| "gfx950".into());
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into());

    let mut srcs: Vec<(PathBuf, &str)> = Vec::new();
    for s in sources(&pkg.join("csrc"), "hip") {
        srcs.push((s, "csrc"));
    }
    for s in sources(&pkg.join("csrc"), "cpp") {
        srcs.push((s, "csrc"));
    }
    for s in sources(&pkg.join("host"), "cpp") {
        srcs.push((s, "host"));
    }
    println!("cargo:rerun-if-changed={}", root.join("include").display());
    println!("cargo:rerun-if-changed={}", pkg.join("csrc").display());
    println!("cargo:rerun-if-changed={}", pkg.join("host").display());
    println!("cargo:rerun-if-env-changed=HIPCC");
    println!("cargo:rerun-if-env-changed=OXIDE_OFFLOAD_ARCH");

    // One hipcc per source, all running at once (paged_decode.hip dominates).
    let mut jobs: Vec<(Child, PathBuf)> = Vec::new();
    let mut objs: Vec<PathBuf> = Vec::new();
    for (src, dir) in &srcs {
        let obj = out.join(format!("{}_{}.o", dir, src.file_stem().unwrap().to_string_lossy()));
        let mut cmd = Command::new(&hipcc);
        cmd.args(["-O3", "-std=c++17", "-fPIC"])
            .arg(format!("--offload-arch={arch}"))
            .args(["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"])
            .arg("-I").arg(root.join("include"))
            .arg("-I").arg(pkg.join("csrc"))
            .arg("-I").arg(pkg.join("host"));
        if src.extension().map_or(false, |x| x == "cpp") {
            cmd.args(["-x", "hip"]);
        }
        cmd.arg("-c").arg(src).arg("-o").arg(&obj);
        let child = cmd.spawn().unwrap_or_else(|e| panic!("spawn {hipcc}: {e}"));
        jobs.push((child, src.clone()));
        objs.push(obj);
    }
    for (mut child, src) in jobs {
        let status = child.wait().expect("hipcc");
        assert!(status.success(), "hipcc --offload-arch={arch} failed on {}", src.display());
    }

    let lib = out.join("liboxide_paged_kv.a");
    let _ = std::fs::remove_file(&lib);
    let status = Command::new("ar").arg("rcs").arg(&lib).args(&objs).status().expect("ar");
    assert!(status.success(), "ar failed");

    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=static=oxide_paged_kv");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rustc-link-lib=dylib=stdc++");
}
