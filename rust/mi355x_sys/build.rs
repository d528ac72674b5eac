//! Links `libmi355x_attn.so` and, when PyTorch-ROCm is found, compiles the one-function
//! shim that returns the ATen current HIP stream.
//!
//! * `MI355X_ATTN_LIB_DIR`: directory holding `libmi355x_attn.so` (built by
//!   `python -m llm_infer_rust_amd.build`, or the hipcc line in the repository's
//!   integration guide). Defaults to `../../llm_infer_rust_amd` next to this crate.
//! * `VIRTUAL_ENV`: the Python environment with PyTorch-ROCm, probed as the reference's own
//!   `build.rs` probes PyTorch-CUDA.
use std::{env, path::PathBuf, process::Command};

fn main() {
    println!("cargo:rustc-check-cfg=cfg(has_mi355x)");
    println!("cargo:rustc-check-cfg=cfg(has_mi355x_stream_shim)");
    println!("cargo:rerun-if-env-changed=MI355X_ATTN_LIB_DIR");
    println!("cargo:rerun-if-env-changed=VIRTUAL_ENV");
    println!("cargo:rerun-if-changed=shim/current_stream.cpp");
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let lib_dir = env::var("MI355X_ATTN_LIB_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("../../llm_infer_rust_amd"));
    if !lib_dir.join("libmi355x_attn.so").exists() {
        println!(
            "cargo:warning=libmi355x_attn.so not found in {}; build it first",
            lib_dir.display()
        );
        return;
    }
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-lib=dylib=mi355x_attn");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
    println!("cargo:rustc-cfg=has_mi355x");

    // ATen's current stream comes from libtorch (c10_hip), as in the reference's bridges.
    let python = env::var("VIRTUAL_ENV")
        .map(|venv| format!("{venv}/bin/python"))
        .unwrap_or_else(|_| "python".to_owned());
    let Ok(output) = Command::new(python)
        .args([
            "-c",
            "import sys, torch; from pathlib import Path; from torch.utils.cpp_extension import include_paths; sys.exit(2) if not torch.version.hip else None; print(int(torch._C._GLIBCXX_USE_CXX11_ABI)); print(Path(torch.__file__).parent / 'lib'); print(*include_paths(device_type='cuda'), sep='\\n')",
        ])
        .output()
    else {
        return;
    };
    if !output.status.success() {
        return;
    }
    let stdout = String::from_utf8_lossy(&output.stdout);
    let mut lines = stdout.lines();
    let abi = lines.next().unwrap_or("0").to_owned();
    let torch_lib = lines.next().unwrap_or_default().to_owned();
    let mut shim = cc::Build::new();
    shim.cpp(true)
        .file("shim/current_stream.cpp")
        .flag_if_supported("-std=c++17")
        .define("_GLIBCXX_USE_CXX11_ABI", abi.as_str())
        .define("USE_ROCM", None)
        .define("__HIP_PLATFORM_AMD__", None)
        .include("/opt/rocm/include")
        .warnings(false);
    for include in lines {
        shim.include(include);
    }
    shim.compile("mi355x_stream_shim");
    println!("cargo:rustc-link-search=native={torch_lib}");
    println!("cargo:rustc-link-lib=dylib=c10_hip");
    println!("cargo:rustc-link-lib=dylib=c10");
    println!("cargo:rustc-cfg=has_mi355x_stream_shim");
}
