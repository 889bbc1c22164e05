"""Build recipe for the gfx950 library (and, for tests, the CPU oracle).

``python -m turboadam_amd.build`` compiles ``csrc/tam_step.hip`` with hipcc
into ``turboadam_amd/_build/libturboadam_amd.so``.  Flags:
  -ffp-contract=off      no implicit fma: every fma in the kernels is explicit,
                         matching where the reference's torch ops fuse;
  -packed-fp32-ops off   no v_pk_*_f32 (hipcc would otherwise form them);
  default fp32 div/sqrt  hipcc's correctly rounded divide and square root.
"""

import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(BUILD_DIR, "libturboadam_amd.so")
SOURCES = [os.path.join(PKG_DIR, "csrc", "tam_step.hip")]
# streaming kernels that bench.py times as the bandwidth ceiling (not part of the library's ABI)
STREAM_LIB_PATH = os.path.join(BUILD_DIR, "libtam_stream.so")
STREAM_SOURCES = [os.path.join(PKG_DIR, "csrc", "tam_stream.hip")]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO_DIR, "include"),
]


def _hipcc(sources, out: str, verbose: bool, extra=()) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    tmp = out + ".tmp"
    cmd = [HIPCC, *HIP_FLAGS, *extra, "-o", tmp, *sources]
    if verbose:
        print(" ".join(cmd))
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr}")
    os.replace(tmp, out)
    return out


def build_library(verbose: bool = False) -> str:
    """The optimizer library, the host module of steady steps and the
    streaming-kernel library bench.py uses."""
    _hipcc(STREAM_SOURCES, STREAM_LIB_PATH, verbose)
    build_host_module(verbose)
    return _hipcc(SOURCES, LIB_PATH, verbose)


# The host side of a steady step in C++ (csrc/tam_host.cpp), a torch extension
# module imported from _build/host by turboadam_amd.optimizer.
HOST_BUILD_DIR = os.path.join(BUILD_DIR, "host")
HOST_SOURCES = [os.path.join(PKG_DIR, "csrc", "tam_host.cpp")]
HOST_MODULE_PATH = os.path.join(HOST_BUILD_DIR, "_tam_host.so")


def build_host_module(verbose: bool = False) -> str:
    """Compile csrc/tam_host.cpp against torch's C++ API (the CPU compiler;
    no device code)."""
    from torch.utils import cpp_extension

    os.makedirs(HOST_BUILD_DIR, exist_ok=True)
    for name in ("_tam_host.so", "tam_host.o"):  # compile every time, as the other libraries
        path = os.path.join(HOST_BUILD_DIR, name)
        if os.path.exists(path):
            os.remove(path)
    cpp_extension.load(name="_tam_host", sources=HOST_SOURCES, build_directory=HOST_BUILD_DIR,
                       extra_cflags=["-O2"], verbose=verbose)
    return HOST_MODULE_PATH


# A measurement build of the same sources that counts the fast paths' exact
# fallbacks (TAM_STATS; read by bench.py --fallback-stats); never the library
# the optimizer loads.
STATS_LIB_PATH = os.path.join(BUILD_DIR, "libturboadam_amd_stats.so")


def build_stats_library(verbose: bool = False) -> str:
    return _hipcc(SOURCES, STATS_LIB_PATH, verbose, ["-DTAM_STATS=1"])


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
    if "--stats" in sys.argv:
        print(build_stats_library(verbose="-v" in sys.argv))
