//! Compiles every HIP source of the library for gfx950 with hipcc and links
//! the shared library, the way burn-mamba_amd/build.py does for the Python
//! binding: one object per source (with that file's extra flags), then one
//! `-shared` link.  HIPCC overrides the compiler path.

use std::env;
use std::path::{Path, PathBuf};
use std::process::Command;

/// Extra flags per source file: MFMA results kept in VGPRs on the MFMA kernels
/// (the same table as burn-mamba_amd/build.py's FILE_FLAGS).
const FILE_FLAGS: &[(&str, &[&str])] = &[
    ("ssd2_mfma.hip", &["-mllvm", "-amdgpu-mfma-vgpr-form"]),
    ("ssd3_mfma.hip", &["-mllvm", "-amdgpu-mfma-vgpr-form"]),
    ("mamba3_fused.hip", &["-mllvm", "-amdgpu-mfma-vgpr-form"]),
    ("lin.hip", &["-mllvm", "-amdgpu-mfma-vgpr-form"]),
];

fn main() {
    let root = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap()).join("../..");
    let csrc = root.join("burn-mamba_amd/csrc");
    let include = root.join("include");
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".into());
    let common = [
        "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
        // no packed-FP32 VALU instructions in any device pass
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    ];
    let mut srcs: Vec<PathBuf> = std::fs::read_dir(&csrc)
        .unwrap()
        .filter_map(|e| e.ok().map(|e| e.path()))
        .filter(|p| p.extension().map_or(false, |x| x == "hip"))
        .collect();
    srcs.sort();
    let mut objs = Vec::new();
    for src in &srcs {
        let name = src.file_name().unwrap().to_str().unwrap();
        let obj = out.join(format!("{name}.o"));
        let extra: &[&str] = FILE_FLAGS.iter().find(|(f, _)| *f == name).map_or(&[], |(_, x)| *x);
        let st = Command::new(&hipcc)
            .args(common)
            .args(extra)
            .arg("-I").arg(&include)
            .arg("-I").arg(&csrc)
            .arg("-c").arg(src)
            .arg("-o").arg(&obj)
            .status()
            .expect("hipcc not found (set HIPCC)");
        assert!(st.success(), "hipcc failed on {}", src.display());
        objs.push(obj);
        println!("cargo:rerun-if-changed={}", src.display());
    }
    // every header the sources include, found the same way as the sources
    let mut headers: Vec<PathBuf> = std::fs::read_dir(&csrc)
        .unwrap()
        .filter_map(|e| e.ok().map(|e| e.path()))
        .filter(|p| p.extension().map_or(false, |x| x == "h"))
        .collect();
    headers.sort();
    for h in &headers {
        let p: &Path = h;
        println!("cargo:rerun-if-changed={}", p.display());
    }
    println!("cargo:rerun-if-changed={}", include.join("mamba_hip.h").display());
    let lib = out.join("libmamba_hip.so");
    let st = Command::new(&hipcc)
        .args(["--offload-arch=gfx950", "-shared", "-fPIC", "-o"])
        .arg(&lib)
        .args(&objs)
        .status()
        .expect("hipcc not found (set HIPCC)");
    assert!(st.success(), "link of libmamba_hip.so failed");
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=mamba_hip");
}
