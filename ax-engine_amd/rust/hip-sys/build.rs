//! Builds libax_hip_sampler.so for gfx950 with hipcc and generates the FFI
//! bindings from include/ax_hip_sampler.h with bindgen.
//!
//! Environment:
//!   AX_HIP_SAMPLER_SRC   directory holding axs_sampler.hip and its headers
//!                        (default: ../../csrc next to this crate)
//!   AX_HIP_SAMPLER_INC   directory holding ax_hip_sampler.h
//!                        (default: ../../../include)
//!   HIPCC / ROCM_PATH    the HIP compiler (default: $ROCM_PATH/bin/hipcc,
//!                        then /opt/rocm/bin/hipcc)
//!   AX_HIP_OFFLOAD_ARCH  GPU target (default: gfx950)
use std::path::PathBuf;
use std::process::Command;

fn env_path(name: &str, default: PathBuf) -> PathBuf {
    println!("cargo:rerun-if-env-changed={name}");
    std::env::var_os(name).map(PathBuf::from).unwrap_or(default)
}

fn main() {
    let manifest = PathBuf::from(std::env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR"));
    let src_dir = env_path("AX_HIP_SAMPLER_SRC", manifest.join("../../csrc"));
    let inc_dir = env_path("AX_HIP_SAMPLER_INC", manifest.join("../../../include"));
    let rocm = env_path("ROCM_PATH", PathBuf::from("/opt/rocm"));
    let hipcc = env_path("HIPCC", rocm.join("bin/hipcc"));
    println!("cargo:rerun-if-env-changed=AX_HIP_OFFLOAD_ARCH");
    let arch = std::env::var("AX_HIP_OFFLOAD_ARCH").unwrap_or_else(|_| String::from("gfx950"));
    let out_dir = PathBuf::from(std::env::var("OUT_DIR").expect("OUT_DIR"));
    let lib = out_dir.join("libax_hip_sampler.so");

    // --- Compile the HIP library ---
    // The flags are the library's own: no FP contraction (the sampling law
    // is reproduced operation by operation), denormals kept, and no packed
    // FP32 instructions.
    let status = Command::new(&hipcc)
        .arg(format!("--offload-arch={arch}"))
        .args(["-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off"])
        .arg("-fno-gpu-flush-denormals-to-zero")
        .args(["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"])
        .arg(format!("-I{}", inc_dir.display()))
        .arg("-o")
        .arg(&lib)
        .arg(src_dir.join("axs_sampler.hip"))
        .status()
        .unwrap_or_else(|e| panic!("cannot run {}: {e}", hipcc.display()));
    assert!(status.success(), "hipcc failed to build libax_hip_sampler.so");

    // --- Link ---
    println!("cargo:rustc-link-search=native={}", out_dir.display());
    println!("cargo:rustc-link-lib=dylib=ax_hip_sampler");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", out_dir.display());
    // exported as DEP_AX_HIP_SAMPLER_LIB_DIR (links = "ax_hip_sampler") so
    // dependents that build executables can embed the same rpath
    println!("cargo:lib_dir={}", out_dir.display());

    // --- Rerun triggers ---
    println!("cargo:rerun-if-changed=build.rs");
    for f in [
        "axs_sampler.hip",
        "axs_device.h",
        "axs_exact_sum.h",
        "axs_expf.h",
        "axs_lm_head.h",
    ] {
        println!("cargo:rerun-if-changed={}", src_dir.join(f).display());
    }
    let header = inc_dir.join("ax_hip_sampler.h");
    println!("cargo:rerun-if-changed={}", header.display());

    // --- Bindings ---
    let bindings = bindgen::Builder::default()
        .header(header.to_string_lossy())
        .allowlist_function("axs_.*")
        .allowlist_type("axs_.*")
        .allowlist_var("AXS_.*")
        .generate()
        .expect("Unable to generate ax_hip_sampler bindings");
    bindings
        .write_to_file(out_dir.join("bindings.rs"))
        .expect("Couldn't write bindings");
}
