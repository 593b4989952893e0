//! Builds libjanus_hip.so from the HIP sources with hipcc for gfx950 (one
//! object per source, packed-FP32 instructions off, as janus_amd/build.py
//! does) and links it. JANUS_HIP_SRC overrides the source directory;
//! JANUS_HIP_LIB_DIR links a library built elsewhere instead.
use std::{env, path::PathBuf, process::Command};

fn main() {
    println!("cargo:rerun-if-env-changed=JANUS_HIP_SRC");
    println!("cargo:rerun-if-env-changed=JANUS_HIP_LIB_DIR");
    if let Ok(dir) = env::var("JANUS_HIP_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-lib=dylib=janus_hip");
        return;
    }
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let src = env::var("JANUS_HIP_SRC").map(PathBuf::from).unwrap_or(manifest.join("../../janus_amd/csrc"));
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".into());
    let mut objs = Vec::new();
    for entry in std::fs::read_dir(&src).expect("HIP source directory") {
        let p = entry.unwrap().path();
        println!("cargo:rerun-if-changed={}", p.display());
        if p.extension().is_some_and(|e| e == "hip") {
            let o = out.join(p.file_stem().unwrap()).with_extension("o");
            let ok = Command::new(&hipcc)
                .args(["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-munsafe-fp-atomics"])
                .args(["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-c"])
                .arg(&p)
                .arg("-o")
                .arg(&o)
                .status()
                .expect("hipcc")
                .success();
            assert!(ok, "hipcc failed on {}", p.display());
            objs.push(o);
        }
    }
    let lib = out.join("libjanus_hip.so");
    let ok = Command::new(&hipcc)
        .args(["--offload-arch=gfx950", "-shared", "-fPIC", "-o"])
        .arg(&lib)
        .args(&objs)
        .status()
        .expect("hipcc link")
        .success();
    assert!(ok, "link failed");
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=janus_hip");
}
