//! Builds libvoxrt_hip.so for gfx950 from the HIP sources in voxrt_amd/csrc with hipcc, into OUT_DIR, and links it.
//!
//! The flags are the ones the numerics depend on (the same as voxrt_amd/build.py):
//!   -ffp-contract=off                  every a*b+c stays two rounded operations, as voxrt's Rust code computes it
//!   -fno-gpu-flush-denormals-to-zero   fp32 denormals kept (IEEE), as on the CPU
//!   -target-feature -packed-fp32-ops   no packed fp32 instructions
//! Environment: HIPCC (default /opt/rocm/bin/hipcc), VOXRT_HIP_SRC (default ../../csrc next to this crate),
//! VOXRT_HIP_ARCH (default gfx950).
use std::env;
use std::path::{Path, PathBuf};
use std::process::Command;

const SOURCES: &[&str] = &[
    "vx_abi.hip",
    "vx_weights.hip",
    "vx_quant.hip",
    "vx_gemm.hip",
    "vx_gemm_stream.hip",
    "vx_gemm_stream_g.hip",
    "vx_gemm_small.hip",
    "vx_glue.hip",
    "vx_attn.hip",
    "vx_encoder.hip",
];

fn run(cmd: &mut Command, what: &str) {
    let status = cmd
        .status()
        .unwrap_or_else(|e| panic!("voxrt-hip-sys: cannot run {what}: {e} (set HIPCC to hipcc's path)"));
    if !status.success() {
        panic!("voxrt-hip-sys: {what} failed with {status}");
    }
}

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let src = env::var("VOXRT_HIP_SRC")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("../../csrc"));
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".to_string());
    let arch = env::var("VOXRT_HIP_ARCH").unwrap_or_else(|_| "gfx950".to_string());
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());
    let flags: Vec<String> = [
        format!("--offload-arch={arch}"),
        "-O3".into(),
        "-std=c++17".into(),
        "-fPIC".into(),
        "-ffp-contract=off".into(),
        "-fno-gpu-flush-denormals-to-zero".into(),
        "-fno-fast-math".into(),
        "-Xclang".into(),
        "-target-feature".into(),
        "-Xclang".into(),
        "-packed-fp32-ops".into(),
    ]
    .into();
    let mut objs = Vec::new();
    for s in SOURCES {
        let path = src.join(s);
        println!("cargo:rerun-if-changed={}", path.display());
        let obj = out.join(Path::new(s).with_extension("o"));
        run(
            Command::new(&hipcc).args(&flags).arg("-c").arg(&path).arg("-o").arg(&obj),
            &format!("hipcc {s}"),
        );
        objs.push(obj);
    }
    for h in ["vx_internal.h", "vx_gemm.h"] {
        println!("cargo:rerun-if-changed={}", src.join(h).display());
    }
    println!("cargo:rerun-if-changed={}", src.join("../../include/voxrt_hip.h").display());
    let lib = out.join("libvoxrt_hip.so");
    run(
        Command::new(&hipcc)
            .arg(format!("--offload-arch={arch}"))
            .args(["-shared", "-fPIC"])
            .args(&objs)
            .arg("-o")
            .arg(&lib),
        "hipcc (link libvoxrt_hip.so)",
    );
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=voxrt_hip");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // the library sits in OUT_DIR: found at run time without LD_LIBRARY_PATH
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", out.display());
    println!("cargo:rerun-if-env-changed=HIPCC");
    println!("cargo:rerun-if-env-changed=VOXRT_HIP_SRC");
    println!("cargo:rerun-if-env-changed=VOXRT_HIP_ARCH");
}
