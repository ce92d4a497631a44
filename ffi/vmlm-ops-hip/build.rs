//! Links libvmlm_hip.so. VMLM_HIP_LIB_DIR names the directory that holds it
//! (sparrow_amd/ after `python -m sparrow_amd.build`); the run-time loader
//! finds it through the same directory in the rpath.
fn main() {
    let dir = std::env::var("VMLM_HIP_LIB_DIR")
        .expect("set VMLM_HIP_LIB_DIR to the directory of libvmlm_hip.so");
    println!("cargo:rerun-if-env-changed=VMLM_HIP_LIB_DIR");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=vmlm_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
}
