// Link libqbk.so.  QBK_LIB_DIR names the directory holding it (default: the
// package directory two levels up, where quantibbler_amd/build.py writes it).
fn main() {
    let dir = std::env::var("QBK_LIB_DIR").unwrap_or_else(|_| {
        let here = std::env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR");
        format!("{here}/../..")
    });
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=qbk");
    println!("cargo:rerun-if-env-changed=QBK_LIB_DIR");
}
