"""The C ABI from a C++ caller with no torch and no Python binding (GPU).

tests/capi/step_check (built by __graft_entry__.build()) fills TamTensor
descriptors itself, runs tam_prepare and tam_multi_tensor_step on hipMalloc'd
state for three steps, and compares parameters and every state array byte for
byte with the CPU oracle after each step.
"""

import os
import subprocess

import pytest

from tests.helpers import log

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "capi", "_build", "step_check")


def test_c_abi_caller_matches_oracle():
    if not os.path.exists(EXE):
        raise RuntimeError(f"{EXE} not built: run __graft_entry__.build()")
    res = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    log(res.stdout.strip())
    assert res.returncode == 0, res.stdout + res.stderr
    assert "capi: ok" in res.stdout
