"""Build recipe of tests/capi/step_check (a test checker, not product): the C-ABI
caller compiled with g++ against the HIP runtime, linked with the CPU oracle
(gcc, -ffp-contract=off) and with turboadam_amd/_build/libturboadam_amd.so."""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
BUILD_DIR = os.path.join(HERE, "_build")
EXE = os.path.join(BUILD_DIR, "step_check")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed ({res.returncode}):\n{res.stderr}")


def build_capi() -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    obj = os.path.join(BUILD_DIR, "tam_oracle.o")
    _run(["gcc", "-O2", "-std=c11", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-c",
          os.path.join(REPO, "oracle", "tam_oracle.c"), "-o", obj])
    lib_dir = os.path.join(REPO, "turboadam_amd", "_build")
    tmp = EXE + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
          os.path.join(HERE, "step_check.cpp"), obj, "-o", tmp,
          "-L", lib_dir, "-lturboadam_amd", "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-lm",
          "-Wl,-rpath,$ORIGIN/../../../turboadam_amd/_build", "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    os.replace(tmp, EXE)
    return EXE


if __name__ == "__main__":
    print(build_capi())
