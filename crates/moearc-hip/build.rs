//! Builds libmoearc_attn.so and its gfx950 code object from ../../moearc_amd/csrc into OUT_DIR,
//! with the commands moearc_amd/build.py runs, and links the crate against it.
//!
//! The linking contract is the reference crate's (crates/moearc-kernels/build.rs:95-112): one
//! dylib, its soname the absolute path of the built object, so a downstream binary's DT_NEEDED
//! names that path and resolves without an rpath of its own. The code object is written beside the
//! library, where the library's context looks for it (MOEARC_CODE_OBJECT overrides).

use std::path::{Path, PathBuf};
use std::process::Command;

fn run(cmd: &mut Command, what: &str) {
    let status = cmd.status().unwrap_or_else(|e| panic!("failed to run {what}: {e}"));
    assert!(status.success(), "{what} failed");
}

fn main() {
    let manifest = PathBuf::from(std::env::var("CARGO_MANIFEST_DIR").unwrap());
    let repo = manifest.join("../..");
    let csrc = repo.join("moearc_amd/csrc");
    let include = repo.join("include");
    let out = PathBuf::from(std::env::var("OUT_DIR").unwrap());
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into());
    println!("cargo:rerun-if-changed={}", csrc.display());
    println!("cargo:rerun-if-changed={}", include.display());
    println!("cargo:rerun-if-env-changed=ROCM_PATH");

    // Device code: every kernel, one translation unit, gfx950 only. Packed-FP32 instructions
    // disabled; MFMA accumulators in VGPRs; the first 14 kernel-argument dwords preloaded.
    let co = out.join("moearc_attn_gfx950.co");
    run(
        Command::new(Path::new(&rocm).join("bin/hipcc"))
            .args(["--offload-arch=gfx950", "--genco", "--no-gpu-bundle-output", "-O3", "-std=c++17"])
            .args(["-fno-honor-nans", "-mllvm", "-amdgpu-mfma-vgpr-form=1"])
            .args(["-mllvm", "-amdgpu-kernarg-preload-count=14"])
            .args(["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"])
            .arg("-I")
            .arg(&csrc)
            .arg(csrc.join("moearc_kernels.hip"))
            .arg("-o")
            .arg(&co),
        "hipcc",
    );

    // Host runtime: the C ABI, against the HIP runtime API only.
    let so = out.join("libmoearc_attn.so");
    run(
        Command::new(std::env::var("CXX").unwrap_or_else(|_| "g++".into()))
            .args(["-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__"])
            .arg("-I")
            .arg(&include)
            .arg("-I")
            .arg(&csrc)
            .arg("-I")
            .arg(Path::new(&rocm).join("include"))
            .arg(csrc.join("runtime.cpp"))
            .arg(csrc.join("kv_cache.cpp"))
            .arg("-o")
            .arg(&so)
            .arg(format!("-Wl,-soname,{}", so.display()))
            .arg("-Wl,--enable-new-dtags")
            .arg(format!("-Wl,-rpath,{}", Path::new(&rocm).join("lib").display()))
            .arg("-L")
            .arg(Path::new(&rocm).join("lib"))
            .args(["-lamdhip64", "-ldl"]),
        "g++",
    );

    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=moearc_attn");
    println!("cargo:rustc-link-search=native={}", Path::new(&rocm).join("lib").display());
    println!("cargo:rustc-env=MOEARC_ATTN_LIB={}", so.display());
}
