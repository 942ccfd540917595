//! Builds libffai_attn.so for gfx950 from the repository's sources, as ffai_amd/build.py does,
//! and links it. FFAI_AMD_ROOT points at the repository (default: two levels up);
//! FFAI_AMD_PREBUILT at an already built libffai_attn.so directory (the compile step is then
//! skipped). Needs ROCm's hipcc and hipBLASLt.

use std::path::{Path, PathBuf};
use std::process::Command;

const SOURCES: [&str; 12] = [
    "fwd_bf16.hip", "fwd_f16.hip", "fwd_f32.hip", "decode.hip", "decode_f16.hip", "decode_vec.hip",
    "kv_cache.hip",
    "gemv.hip", "probe.hip", "attn_launch.hip", "attn_api.cpp", "encoder_attn.cpp",
];

fn hipcc() -> PathBuf {
    if let Ok(p) = std::env::var("HIPCC") {
        return PathBuf::from(p);
    }
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into());
    Path::new(&rocm).join("bin").join("hipcc")
}

fn main() {
    println!("cargo:rerun-if-env-changed=FFAI_AMD_ROOT");
    println!("cargo:rerun-if-env-changed=FFAI_AMD_PREBUILT");
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into());
    if let Ok(dir) = std::env::var("FFAI_AMD_PREBUILT") {
        println!("cargo:rustc-link-search=native={dir}");
    } else {
        let manifest = PathBuf::from(std::env::var("CARGO_MANIFEST_DIR").unwrap());
        let root = std::env::var("FFAI_AMD_ROOT")
            .map(PathBuf::from)
            .unwrap_or_else(|_| manifest.join("..").join(".."));
        let csrc = root.join("ffai_amd").join("csrc");
        let include = root.join("include");
        let out = PathBuf::from(std::env::var("OUT_DIR").unwrap());
        let mut objs = Vec::new();
        for src in SOURCES {
            let obj = out.join(format!("{src}.o"));
            // The flags of ffai_amd/build.py: gfx950 only, packed-FP32 VALU ops off, and the
            // NaN-free assumptions for device code only (host argument checks see NaN as NaN).
            let status = Command::new(hipcc())
                .args(["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950"])
                .args(["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"])
                .args(["-Xarch_device", "-fno-honor-nans", "-Xarch_device", "-mno-amdgpu-ieee"])
                .arg("-I").arg(&include)
                .args(["-c", "-x", "hip"]).arg(csrc.join(src))
                .arg("-o").arg(&obj)
                .status()
                .expect("hipcc not found: set HIPCC or ROCM_PATH");
            assert!(status.success(), "hipcc failed on {src}");
            objs.push(obj);
            println!("cargo:rerun-if-changed={}", csrc.join(src).display());
        }
        for dep in std::fs::read_dir(&csrc).unwrap().chain(std::fs::read_dir(&include).unwrap()) {
            println!("cargo:rerun-if-changed={}", dep.unwrap().path().display());
        }
        let status = Command::new(hipcc())
            .args(["--offload-arch=gfx950", "-shared", "-fPIC", "-o"])
            .arg(out.join("libffai_attn.so"))
            .args(&objs)
            .arg(format!("-L{rocm}/lib"))
            .args(["-lhipblaslt", &format!("-Wl,-rpath,{rocm}/lib")])
            .status()
            .expect("hipcc not found");
        assert!(status.success(), "linking libffai_attn.so failed");
        println!("cargo:rustc-link-search=native={}", out.display());
    }
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=ffai_attn");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rustc-link-lib=dylib=hipblaslt");
}
