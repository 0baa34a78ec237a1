// Links librtq.so (built in-tree by `python -c "import __graft_entry__ as g; g.build()"`, one
// directory up from this crate) and the HIP runtime it needs.  RTQ_LIB_DIR overrides the location.
fn main() {
    let dir = std::env::var("RTQ_LIB_DIR").unwrap_or_else(|_| {
        let here = std::path::PathBuf::from(std::env::var("CARGO_MANIFEST_DIR").unwrap());
        here.parent().unwrap().to_string_lossy().into_owned()
    });
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rerun-if-env-changed=RTQ_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=rtq");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}:{rocm}/lib");
}
