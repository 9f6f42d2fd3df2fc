// build.rs of candelora-metal-kernels with the `rocm` feature (Cargo.toml:
// `[features] rocm = []`): builds libcmk_iq2.so for gfx950 with hipcc through
// candelora-metal-kernels_amd/build.py and links it.  Not built here.
fn main() {
    if std::env::var_os("CARGO_FEATURE_ROCM").is_none() { return; }
    let pkg = std::path::Path::new(env!("CARGO_MANIFEST_DIR")).join("candelora-metal-kernels_amd");
    let ok = std::process::Command::new("python3").arg(pkg.join("build.py"))
        .status().map(|s| s.success()).unwrap_or(false);
    assert!(ok, "building libcmk_iq2.so (hipcc --offload-arch=gfx950) failed");
    println!("cargo:rustc-link-search=native={}", pkg.display());
    println!("cargo:rustc-link-lib=dylib=cmk_iq2");
    println!("cargo:rerun-if-changed={}", pkg.join("csrc").display());
}
