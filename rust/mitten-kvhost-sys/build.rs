//! Links the prebuilt host bookkeeping library (`libmitten_kvhost.so`, g++,
//! no GPU needed), from the same directory as the device library.
fn main() {
    let dir = std::env::var("MITTEN_KV_LIB_DIR").expect("set MITTEN_KV_LIB_DIR to the directory of libmitten_kvhost.so");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=mitten_kvhost");
    println!("cargo:rerun-if-env-changed=MITTEN_KV_LIB_DIR");
}
