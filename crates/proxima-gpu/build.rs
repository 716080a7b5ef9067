//! Links libproxima_hip.so (built by `python proxima_amd/build.py` with hipcc
//! for gfx950). `PROXIMA_HIP_LIB_DIR` names its directory; the default is
//! where a packaged install puts it.

fn main() {
    let dir = std::env::var("PROXIMA_HIP_LIB_DIR").unwrap_or_else(|_| "/opt/proxima-hip/lib".to_owned());
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=proxima_hip");
    println!("cargo:rerun-if-env-changed=PROXIMA_HIP_LIB_DIR");
}
