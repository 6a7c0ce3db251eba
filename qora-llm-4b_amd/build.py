"""Build recipe for libqora_mixer.so and its gfx950 code objects.

    python qora-llm-4b_amd/build.py          # build into qora-llm-4b_amd/lib/

Each csrc/<name>.hip becomes lib/qm_<name>.hsaco (hipcc --genco for gfx950;
loaded at run time with hipModuleLoad), and csrc/qm_runtime.cpp becomes
lib/libqora_mixer.so (host code only, g++ against the HIP runtime).  The
products are git-ignored and travel with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
ROOT = PKG.parent
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "--genco", "-O3", "-std=c++17",
    # Keep the compiler from emitting packed-fp32 VALU ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in arch VGPRs: no AGPR<->VGPR copies around VALU work on
    # the accumulators.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-parameter",
]

KERNELS = ["dn_decode", "gqa_decode", "util", "dn_prefill", "gqa_prefill", "q4_proj", "q4_vocab", "sample"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def hip_cmd(name: str) -> list[str]:
    return [str(ROCM / "bin" / "hipcc"), *HIPCC_FLAGS, "-I", str(CSRC),
            str(CSRC / f"{name}.hip"), "-o", str(LIB / f"qm_{name}.hsaco")]


def noalloc_cmd() -> list[str]:
    """csrc/qm_noalloc.hip, the fixed device scratch of the allocation-free
    entry point, compiled into an object of the host library itself (its
    device array lives in the library's own gfx950 fat binary)."""
    flags = [f for f in HIPCC_FLAGS if f != "--genco"]
    return [str(ROCM / "bin" / "hipcc"), *flags, "-fPIC", "-c", "-I", str(CSRC),
            str(CSRC / "qm_noalloc.hip"), "-o", str(LIB / "qm_noalloc.o")]


def host_cmd() -> list[str]:
    return ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
            "-Wall", "-Wextra", "-Wno-unused-result", "-D__HIP_PLATFORM_AMD__",
            "-I", str(ROOT / "include"), "-I", str(CSRC), "-I", str(ROCM / "include"),
            str(CSRC / "qm_runtime.cpp"), str(LIB / "qm_noalloc.o"), "-o", str(LIB / "libqora_mixer.so"),
            f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}", "-ldl"]


def build(jobs: int = 8) -> None:
    LIB.mkdir(exist_ok=True)
    cmds = [hip_cmd(k) for k in KERNELS] + [noalloc_cmd()]
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for f in [ex.submit(_run, c) for c in cmds]:
            f.result()
    _run(host_cmd())


def build_oracle() -> None:
    _run(["make", "-s", "-C", str(ROOT / "oracle")])


def build_host_test() -> None:
    """tests/cpp/host_mirror_test.cpp: the C++ mirror driven against the oracle
    (test infrastructure; needs the library and the oracle built)."""
    _run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-I", str(ROOT / "include"),
          "-I", str(PKG / "host"), "-I", str(ROOT / "oracle"), "-I", str(ROOT / "tests" / "cpp"),
          str(ROOT / "tests" / "cpp" / "host_mirror_test.cpp"), "-o", str(LIB / "host_mirror_test"),
          f"-L{LIB}", "-lqora_mixer", f"-L{ROOT / 'oracle'}", "-loracle",
          "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,$ORIGIN/../../oracle"])



def build_file_test() -> None:
    """tests/cpp/qor4b_file_test.cpp: the .qor4b parser on the CPU (g++ only,
    no device code; test infrastructure)."""
    _run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-I", str(PKG / "host"), "-I", str(ROOT / "tests" / "cpp"),
          str(ROOT / "tests" / "cpp" / "qor4b_file_test.cpp"), "-o", str(LIB / "qor4b_file_test")])


def build_plan_test() -> None:
    """tests/cpp/gqa_plan_test.cpp: the GQA prefill row-block order on the CPU
    (g++ only, no device code; test infrastructure)."""
    _run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-I", str(CSRC),
          str(ROOT / "tests" / "cpp" / "gqa_plan_test.cpp"), "-o", str(LIB / "gqa_plan_test")])


if __name__ == "__main__":
    build()
    if "--no-oracle" not in sys.argv:
        build_oracle()
        build_host_test()
        build_file_test()
        build_plan_test()
    print("built:", ", ".join(sorted(p.name for p in LIB.iterdir())))
