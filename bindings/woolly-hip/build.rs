// Links libwoolly_hip.so: WOOLLY_HIP_LIB_DIR names the directory that holds it
// (woolly_amd/ after `python -m woolly_amd.build`).
fn main() {
    println!("cargo:rerun-if-env-changed=WOOLLY_HIP_LIB_DIR");
    if let Ok(dir) = std::env::var("WOOLLY_HIP_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
    }
    println!("cargo:rustc-link-lib=dylib=woolly_hip");
}
