// Links libmitok.so the way the transformer crate's build.rs links OpenBLAS
// (build.rs:20-30 of the crate): the directory comes from the environment.
fn main() {
    let dir = std::env::var("MITOK_DIR").expect("MITOK_DIR: the directory holding libmitok.so");
    println!("cargo:rustc-link-search=native={}", dir);
    println!("cargo:rustc-link-lib=dylib=mitok");
    println!("cargo:rerun-if-env-changed=MITOK_DIR");
}
