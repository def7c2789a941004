//! build.rs for native/arm_ai_nif with the `gpu_mi355x` feature: compiles the
//! MI355X library (libarm_ai_amd.so) from its HIP sources with hipcc for
//! gfx950 and links the NIF against it.  Without the feature it does nothing,
//! and the crate builds exactly as before (candle on the CPU).
//!
//! Inputs (environment):
//!   ARM_AI_AMD_CSRC  directory of the library's .hip sources and headers
//!                    (default: ../../arm_ai_amd/csrc from this crate, the
//!                    layout of the arm_ai_amd checkout)
//!   ARM_AI_AMD_LIB_DIR  a directory that already holds libarm_ai_amd.so:
//!                    skip the compile and link against it
//!   HIPCC            the compiler (default /opt/rocm/bin/hipcc)
//!   ARM_AI_AMD_ARCH  the offload target (default gfx950)
//! The .so goes to OUT_DIR and the NIF's RUNPATH points there (and to
//! $ORIGIN, for a release that copies the .so next to the NIF in priv/).
use std::env;
use std::path::{Path, PathBuf};
use std::process::{Child, Command};

// The flags arm_ai_amd/build.py compiles with: IEEE f32 (no fast-math, no
// FMA contraction: the bit-exact quantizers and the f32 epilogues depend on
// it) and the packed-f32 instructions left to the compiler's discretion off.
const HIPCC_FLAGS: &[&str] = &[
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
];

fn main() {
    println!("cargo:rerun-if-env-changed=ARM_AI_AMD_CSRC");
    println!("cargo:rerun-if-env-changed=ARM_AI_AMD_LIB_DIR");
    println!("cargo:rerun-if-env-changed=HIPCC");
    println!("cargo:rerun-if-env-changed=ARM_AI_AMD_ARCH");
    if env::var_os("CARGO_FEATURE_GPU_MI355X").is_none() {
        return;
    }
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    let lib_dir = match env::var("ARM_AI_AMD_LIB_DIR") {
        Ok(dir) => PathBuf::from(dir),
        Err(_) => compile_library(&rocm),
    };
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-lib=dylib=arm_ai_amd");
    // the HIP runtime: the NIF calls it for device buffers and the decode graph
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
    println!("cargo:rustc-link-arg=-Wl,-rpath,$ORIGIN");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{rocm}/lib");
}

fn compile_library(rocm: &str) -> PathBuf {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let csrc = env::var("ARM_AI_AMD_CSRC")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("../../arm_ai_amd/csrc"));
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| format!("{rocm}/bin/hipcc"));
    let arch = env::var("ARM_AI_AMD_ARCH").unwrap_or_else(|_| "gfx950".to_string());
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());

    let mut sources: Vec<PathBuf> = std::fs::read_dir(&csrc)
        .unwrap_or_else(|e| panic!("ARM_AI_AMD_CSRC={}: {e}", csrc.display()))
        .filter_map(|e| e.ok().map(|e| e.path()))
        .filter(|p| p.extension().map_or(false, |x| x == "hip"))
        .collect();
    sources.sort();
    assert!(!sources.is_empty(), "no .hip sources in {}", csrc.display());
    for entry in std::fs::read_dir(&csrc).unwrap().flatten() {
        println!("cargo:rerun-if-changed={}", entry.path().display());
    }

    // one hipcc per translation unit, all running at once
    let mut jobs: Vec<(PathBuf, Child)> = Vec::new();
    let mut objects = Vec::new();
    for src in &sources {
        let obj = out.join(format!("{}.o", src.file_stem().unwrap().to_string_lossy()));
        let child = Command::new(&hipcc)
            .arg(format!("--offload-arch={arch}"))
            .args(HIPCC_FLAGS)
            .arg("-c")
            .arg(src)
            .arg("-o")
            .arg(&obj)
            .spawn()
            .unwrap_or_else(|e| panic!("{hipcc}: {e}"));
        jobs.push((src.clone(), child));
        objects.push(obj);
    }
    for (src, mut child) in jobs {
        let status = child.wait().expect("hipcc");
        assert!(status.success(), "hipcc failed on {}", src.display());
    }
    let lib = out.join("libarm_ai_amd.so");
    link(&hipcc, &arch, &objects, &lib);
    out
}

fn link(hipcc: &str, arch: &str, objects: &[PathBuf], lib: &Path) {
    let status = Command::new(hipcc)
        .arg(format!("--offload-arch={arch}"))
        .arg("-shared")
        .arg("-fPIC")
        .args(objects)
        .arg("-o")
        .arg(lib)
        .status()
        .expect("hipcc link");
    assert!(status.success(), "linking {} failed", lib.display());
}
