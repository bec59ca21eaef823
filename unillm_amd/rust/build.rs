// Builds libunillm_hip.so for gfx950 from the HIP sources beside this crate
// (../csrc) and links it as a dylib.  The same compile and link lines as
// unillm_amd/build.py: one hipcc -c per translation unit, packed-fp32 VALU ops off
// on the device pass, one hipcc -shared link.
//
// Environment:
//   UNILLM_HIP_LIB_DIR  link the libunillm_hip.so in this directory instead of building
//   HIPCC               the compiler (default /opt/rocm/bin/hipcc)
use std::env;
use std::path::PathBuf;
use std::process::Command;

// Keep in step with SOURCES in unillm_amd/build.py (a CPU test compares the two lists).
const SOURCES: &[&str] = &[
    "capi.hip",
    "weights.hip",
    "gemv.hip",
    "decode.hip",
    "prefill.hip",
    "attention.hip",
    "dense.hip",
];

// Libraries the link adds: the dense (F32 / F16 / BF16) weights' f32 GEMM.  Keep in step
// with LIBS in unillm_amd/build.py.
const LIBS: &[&str] = &["-L/opt/rocm/lib", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib"];

const FLAGS: &[&str] = &[
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
];

fn run(cmd: &mut Command, what: &str) {
    let status = cmd
        .status()
        .unwrap_or_else(|e| panic!("{what}: cannot run {:?}: {e}", cmd.get_program()));
    if !status.success() {
        panic!("{what} failed ({status})");
    }
}

fn main() {
    println!("cargo:rerun-if-env-changed=UNILLM_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=HIPCC");
    if let Ok(dir) = env::var("UNILLM_HIP_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-lib=dylib=unillm_hip");
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
        return;
    }
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR"));
    let csrc = manifest.join("..").join("csrc");
    let include = manifest.join("..").join("..").join("include");
    let out = PathBuf::from(env::var("OUT_DIR").expect("OUT_DIR"));
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".to_string());

    println!("cargo:rerun-if-changed={}", csrc.display());
    println!("cargo:rerun-if-changed={}", include.display());
    let mut objs = Vec::new();
    for src in SOURCES {
        let obj = out.join(src.replace(".hip", ".o"));
        run(
            Command::new(&hipcc)
                .args(FLAGS)
                .arg("-c")
                .arg(csrc.join(src))
                .arg("-o")
                .arg(&obj),
            &format!("hipcc {src}"),
        );
        objs.push(obj);
    }
    let lib = out.join("libunillm_hip.so");
    run(
        Command::new(&hipcc)
            .args(["--offload-arch=gfx950", "-shared", "-fPIC", "-o"])
            .arg(&lib)
            .args(&objs)
            .args(LIBS),
        "hipcc -shared",
    );
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=unillm_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", out.display());
}
