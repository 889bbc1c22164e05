"""Build the CPU oracle (test infrastructure only): gcc -> oracle/_build/libtam_oracle.so.

-ffp-contract=off keeps every fp32 operation separately rounded, as torch's
CPU kernels do; -fno-fast-math and -O2 keep IEEE semantics.  -fopenmp runs
the loops over independent blocks and elements on several threads; every
reduction keeps its fixed order, so results do not depend on the thread count.
"""

import os
import subprocess

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
BUILD_DIR = os.path.join(ORACLE_DIR, "_build")
LIB_PATH = os.path.join(BUILD_DIR, "libtam_oracle.so")
SRC = os.path.join(ORACLE_DIR, "tam_oracle.c")


def build_oracle(verbose: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
           "-o", tmp, SRC, "-lm"]
    if verbose:
        print(" ".join(cmd))
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed ({res.returncode}):\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_oracle(verbose=True))
