"""TEST INFRASTRUCTURE ONLY -- deterministic synthetic inputs for parity runs.

Approximately normal values built from Philox4x32-10 uniforms with exact
arithmetic only (Irwin-Hall: the sum of 12 uniforms minus 6, each uniform a
multiple of 2^-24, summed exactly in float64), so every machine produces the
same bits and fixtures need not store their inputs.
"""

import numpy as np

from . import oracle as O

GEN_SEED = 0x6E6F726D616C2121  # separate key from the optimizer's rounding stream


def normal(n: int, stream: int, draw: int, seed: int = GEN_SEED) -> np.ndarray:
    """n approximately N(0,1) float64 values of (stream, draw)."""
    u = O.input_uniforms(stream & 0xFFFFFFFF, draw & 0xFFFFFFFF, seed, 12 * n).astype(np.float64)
    return u.reshape(n, 12).sum(axis=1) - 6.0


def param_init(sizes, scale=0.02, stream0=1000):
    return [(normal(n, stream0 + i, 0) * scale).astype(np.float32) for i, n in enumerate(sizes)]


def grad_sigmas(count, log_center=np.log(1e-3), stream=999):
    z = normal(count, stream, 1)
    return np.exp(log_center + z)


def grads(sizes, step, sigmas, drift_scale=0.3, stream0=2000):
    """g_i = sigma_i * (z + 0.3 d_i): fresh z each step, fixed drift d_i per tensor."""
    out = []
    for i, n in enumerate(sizes):
        z = normal(n, stream0 + i, 1 + step)
        d = normal(n, stream0 + i, 0)
        out.append((sigmas[i] * (z + drift_scale * d)).astype(np.float32))
    return out
