"""The step without a caller workspace (tam_multi_tensor_step_static) equals
the step with one (tam_multi_tensor_step) bit for bit.

Two optimizers take identical parameters and gradients; one issues each step
through tam_multi_tensor_step, the other through tam_multi_tensor_step_static
(both through the C ABI).  A first parameter set runs two steps, then a
second, smaller set runs two more on the same device, so the static scratch
is reused with less of it in use.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import compare_states, from_torch, gpu_state, log, make_grads, to_bits, to_torch

pytestmark = pytest.mark.gpu

F32, BF16, F16 = O.DT_F32, O.DT_BF16, O.DT_F16


def _static_optimizer_class():
    from turboadam_amd import TurboAdam, _lib

    class StaticStep(TurboAdam):
        """Issues each step through the static-scratch entry point."""

        def _issue(self, lib, desc_ptr, arr, info, ws, stream):
            rc = lib.tam_multi_tensor_step_static(desc_ptr, arr, ctypes.byref(info), self.philox_seed, stream)
            _lib.check(rc, "tam_multi_tensor_step_static")

    return TurboAdam, StaticStep


def _bits(a):
    return a.view(np.uint32) if a.dtype == np.float32 else a


def _run_pair(sizes, dts, steps, seed, **kw):
    TurboAdam, StaticStep = _static_optimizer_class()
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(seed)
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
    pa = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    pb = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    oa = TurboAdam(pa, philox_seed=99 + seed, **kw)
    ob = StaticStep(pb, philox_seed=99 + seed, **kw)
    sigmas = np.exp(np.log(1e-3) + rng.standard_normal(len(sizes)))
    bad = []
    for s in range(steps):
        grads = make_grads(rng, sizes, dts, sigmas)
        for p, q, g, dt, n in zip(pa, pb, grads, dts, sizes):
            p.grad = to_torch(g, dt, (n,), dev)
            q.grad = to_torch(g, dt, (n,), dev)
        log(f"sizes {sizes}: step {s + 1}")
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        for i, (p, q) in enumerate(zip(pa, pb)):
            where = f"step {s + 1} tensor {i} (n={sizes[i]})"
            if not np.array_equal(_bits(from_torch(p)), _bits(from_torch(q))):
                bad.append(f"{where}: params differ")
            bad += compare_states(gpu_state(ob, q), gpu_state(oa, p), where)
    return bad


def test_static_scratch_step_equals_workspace_step():
    # first call set: CoState and fp32-m tensors, three dtypes, tails, more
    # than one alpha chunk and selection slice (1.2M elements)
    bad = _run_pair([1_200_000, 70_000, 5000, 4096 * 3 + 5, 300], [BF16, F32, F16, F32, BF16], 2, seed=1,
                    lr=1e-3, weight_decay=0.01)
    assert not bad, "\n".join(bad[:20])
    # second, smaller set on the same device's scratch
    bad = _run_pair([9000, 1000], [F32, BF16], 2, seed=2, lr=2e-3)
    assert not bad, "\n".join(bad[:20])


def test_static_scratch_rejects_a_step_above_its_size():
    from turboadam_amd import _lib

    lib = _lib.load()
    t = _lib.TamTensor()
    t.param, t.grad = 0x10000, 0x20000
    t.n = 1 << 30  # workspace of about 64 MiB + per-tensor histograms: above the scratch
    t.dtype = _lib.TAM_DTYPE_F32
    t.flags = _lib.TAM_FLAG_COSTATE | _lib.TAM_FLAG_COMPRESS_V
    t.v_idx, t.v_scales, t.v_bits = 0x30000, 0x40000, 4
    t.signs = t.labels = t.norms = t.amp = t.alpha = 0x60000
    t.sqrt_block = np.float32(np.sqrt(128.0))
    arr = (_lib.TamTensor * 1)(t)
    info = _lib.TamStepInfo()
    assert lib.tam_prepare(arr, 1, ctypes.byref(info)) == 0
    assert info.ws_bytes > _lib.TAM_STATIC_SCRATCH_BYTES
    rc = lib.tam_multi_tensor_step_static(0x1000, arr, ctypes.byref(info), 0, None)
    assert rc == 2 and "static scratch" in lib.tam_last_error().decode()
