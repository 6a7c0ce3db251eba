//! Builds the gfx950 code objects and the host library the crate links,
//! with the same recipe as qora-llm-4b_amd/build.py:
//!   - each csrc/<kernel>.hip -> $OUT_DIR/qm_<kernel>.hsaco (hipcc --genco),
//!     loaded at run time by qm_create from the directory of the library;
//!   - csrc/qm_noalloc.hip -> an object with its own gfx950 fat binary (the
//!     fixed scratch array of qm_gqa_decode_noalloc);
//!   - csrc/qm_runtime.cpp + that object -> $OUT_DIR/libqora_mixer.so (g++,
//!     linked against libamdhip64).
use std::env;
use std::path::{Path, PathBuf};
use std::process::Command;

const KERNELS: &[&str] = &["dn_decode", "gqa_decode", "util", "dn_prefill", "gqa_prefill", "q4_proj", "q4_vocab", "sample"];

// hipcc flags of every device compile: gfx950 only; no packed-fp32 VALU ops;
// MFMA results in arch VGPRs.
const HIPCC_FLAGS: &[&str] = &[
    "--offload-arch=gfx950", "-O3", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-parameter",
];

fn run(cmd: &mut Command) {
    let status = cmd.status().unwrap_or_else(|e| panic!("cannot run {:?}: {}", cmd, e));
    if !status.success() {
        panic!("build step failed ({}): {:?}", status, cmd);
    }
}

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let pkg = manifest.join("../..");                 // qora-llm-4b_amd/
    let csrc = pkg.join("csrc");
    let include = pkg.join("../include");
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    let hipcc = Path::new(&rocm).join("bin/hipcc");

    for k in KERNELS {
        run(Command::new(&hipcc)
            .args(HIPCC_FLAGS)
            .arg("--genco")
            .arg("-I").arg(&csrc)
            .arg(csrc.join(format!("{}.hip", k)))
            .arg("-o").arg(out.join(format!("qm_{}.hsaco", k))));
    }
    let noalloc = out.join("qm_noalloc.o");
    run(Command::new(&hipcc)
        .args(HIPCC_FLAGS)
        .args(["-fPIC", "-c"])
        .arg("-I").arg(&csrc)
        .arg(csrc.join("qm_noalloc.hip"))
        .arg("-o").arg(&noalloc));
    run(Command::new("g++")
        .args(["-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", "-D__HIP_PLATFORM_AMD__"])
        .arg("-I").arg(&include)
        .arg("-I").arg(&csrc)
        .arg("-I").arg(Path::new(&rocm).join("include"))
        .arg(csrc.join("qm_runtime.cpp"))
        .arg(&noalloc)
        .arg("-o").arg(out.join("libqora_mixer.so"))
        .arg(format!("-L{}/lib", rocm))
        .arg("-lamdhip64")
        .arg(format!("-Wl,-rpath,{}/lib", rocm))
        .arg("-ldl"));

    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=qora_mixer");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", out.display());
    // qm_create(.., NULL, ..) finds the code objects next to the library
    println!("cargo:rustc-env=QORA_MIXER_CODE_OBJECTS={}", out.display());
    println!("cargo:rerun-if-changed={}", csrc.display());
    println!("cargo:rerun-if-changed={}", include.join("qora_mixer.h").display());
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}
