//! Links libcfattn.so, built by `python -c "import cpuforge_amd.build as b; b.build()"` (or the
//! repository's `__graft_entry__.build()`) into `cpuforge_amd/`.  CFATTN_LIB_DIR names that
//! directory; the binary finds the library at run time through the rpath set here.
fn main() {
    let dir = std::env::var("CFATTN_LIB_DIR")
        .expect("set CFATTN_LIB_DIR to the directory that holds libcfattn.so (cpuforge_amd/)");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=cfattn");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    println!("cargo:rerun-if-env-changed=CFATTN_LIB_DIR");
}
