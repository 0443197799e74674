//! Builds libfthip.so -- the gfx950 code objects of every kernel, linked into
//! one shared library with the C ABI of include/ft_hip.h -- from this
//! repository's HIP sources, the way ft-cuda/build.rs compiles its kernels
//! with nvcc (ft-cuda/build.rs:8-14). freetoken-rs_amd/build.py runs
//! `hipcc --offload-arch=gfx950 -O3 -ffp-contract=off ...` per source and links
//! the objects; the crate then links the library by name.
use std::path::PathBuf;
use std::process::Command;

fn main() {
    let pkg = PathBuf::from(env!("CARGO_MANIFEST_DIR")).join("..");
    let status = Command::new("python3")
        .arg(pkg.join("build.py"))
        .status()
        .expect("python3 (and hipcc from ROCm) are needed to build ft-hip");
    assert!(status.success(), "hipcc build of libfthip.so failed");
    println!("cargo:rustc-link-search=native={}", pkg.join("lib").display());
    println!("cargo:rustc-link-lib=dylib=fthip");
    println!("cargo:rerun-if-changed={}", pkg.join("csrc").display());
    println!("cargo:rerun-if-changed={}", pkg.join("../include/ft_hip.h").display());
}
