// Link libiq_qgemm.so (built in-tree by `python -m inferq_amd._build`) and
// the HIP runtime.  INFERQ_AMD_LIB_DIR points at the directory holding the
// library (the repository's inferq_amd/).
fn main() {
    let dir = std::env::var("INFERQ_AMD_LIB_DIR").expect("set INFERQ_AMD_LIB_DIR to the directory of libiq_qgemm.so");
    println!("cargo:rerun-if-env-changed=INFERQ_AMD_LIB_DIR");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=iq_qgemm");
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_owned());
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
}
