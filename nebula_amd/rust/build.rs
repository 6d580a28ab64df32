// build.rs lines for crates/nebula-hydrogen when it links the qgemm module (Linux / ROCm): the
// library is built in-tree by nebula_amd/build.py; NEBULA_HQ_LIB points at its directory.
fn main() {
    let dir = std::env::var("NEBULA_HQ_LIB").unwrap_or_else(|_| "../../nebula_amd/lib".to_string());
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=nebula_hq");
    println!("cargo:rerun-if-env-changed=NEBULA_HQ_LIB");
}
