//! Links the prebuilt device library. `python -m mitten_amd._build` writes
//! `libmitten_kv.so` (hipcc, gfx950) to `mitten_amd/lib/`; point
//! `MITTEN_KV_LIB_DIR` there. The library's RPATH finds the HIP runtime.
fn main() {
    let dir = std::env::var("MITTEN_KV_LIB_DIR").expect("set MITTEN_KV_LIB_DIR to the directory of libmitten_kv.so");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=mitten_kv");
    println!("cargo:rerun-if-env-changed=MITTEN_KV_LIB_DIR");
}
