"""Resuming from checkpoints on the GPU, bit for bit.

* A checkpoint in the reference's format (pickled turboadam.costate managers,
  1Q dicts with rand_buf; reference optimizer.py:238-286) written from the oracle's state
  after some steps, loaded with load_reference_checkpoint, continues exactly as
  the oracle does.
* This package's own state_dict round trip (through torch.save / torch.load)
  continues exactly as an uninterrupted run, including a non-default Philox
  seed.
"""

import io

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import (compare_states, from_torch, gpu_state, log, reference_manager_class,
                           reference_state_dict, to_bits, to_torch)

pytestmark = pytest.mark.gpu

F32, BF16 = O.DT_F32, O.DT_BF16
KW = dict(lr=1e-3, weight_decay=0.05)


def _grads(rng, sizes, dts, steps):
    return [[to_bits((rng.standard_normal(n) * 1e-3).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
            for _ in range(steps)]


def _bits(a):
    return a.view(np.uint32) if a.dtype == np.float32 else a


def test_resume_from_reference_format_checkpoint():
    from turboadam_amd import TurboAdam, load_reference_checkpoint

    sizes, dts = [70_000, 5000, 300], [BF16, F32, F32]
    shapes = [(700, 100), (50, 100), (300,)]
    rng = np.random.default_rng(21)
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
    grads = _grads(rng, sizes, dts, 5)
    seed = 808
    orc = O.OracleTurboAdam([a.copy() for a in init], dtypes=dts, seed=seed, **KW)
    for s in range(3):
        orc.step(grads[s])
    log("reference-format checkpoint after 3 oracle steps")
    buf = io.BytesIO()
    with reference_manager_class() as ref_cls:
        torch.save(reference_state_dict(orc, shapes, ref_cls), buf)
    buf.seek(0)
    sd = load_reference_checkpoint(buf, map_location="cpu")
    dev = torch.device("cuda:0")
    params = [torch.nn.Parameter(to_torch(orc.param_groups[0]["params"][i], dt, shp, dev))
              for i, (dt, shp) in enumerate(zip(dts, shapes))]
    opt = TurboAdam(params, philox_seed=seed, **KW)
    opt.load_state_dict(sd)
    bad = []
    for s in range(3, 5):
        for p, g, dt, shp in zip(params, grads[s], dts, shapes):
            p.grad = to_torch(g, dt, shp, dev)
        opt.step()
        torch.cuda.synchronize()
        orc.step(grads[s])
        for i, p in enumerate(params):
            if not np.array_equal(_bits(from_torch(p)), _bits(orc.param_groups[0]["params"][i])):
                bad.append(f"step {s + 1} tensor {i}: params differ")
            bad += compare_states(gpu_state(opt, p), orc.state[i], f"step {s + 1} tensor {i}")
    assert not bad, "\n".join(bad[:20])


def test_state_dict_round_trip_resumes_bit_identically():
    from turboadam_amd import TurboAdam
    from turboadam_amd.costate import CoStateManager

    # a bf16 tensor below min_m_compress_elements (fp32 exp_avg) and a
    # compress_v=False group (fp32 exp_avg_sq of a bf16 tensor): torch's loader
    # would round those fp32 moments to bf16
    sizes, dts = [70_000, 5000, 300, 300, 6000], [BF16, BF16, F32, BF16, BF16]
    shapes = [(70_000,), (50, 100), (300,), (300,), (60, 100)]
    rng = np.random.default_rng(22)
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
    grads = _grads(rng, sizes, dts, 5)
    dev = torch.device("cuda:0")

    def make():
        return [torch.nn.Parameter(to_torch(a, dt, shp, dev)) for a, dt, shp in zip(init, dts, shapes)]

    def run(opt, params, steps):
        for s in steps:
            for p, g, dt, shp in zip(params, grads[s], dts, shapes):
                p.grad = to_torch(g, dt, shp, dev)
            opt.step()
        torch.cuda.synchronize()

    def groups(params):
        return [{"params": params[:4]}, {"params": params[4:], "compress_v": False}]

    pa = make()
    oa = TurboAdam(groups(pa), philox_seed=31337, **KW)
    run(oa, pa, range(5))
    pb = make()
    ob = TurboAdam(groups(pb), philox_seed=31337, **KW)
    run(ob, pb, range(3))
    buf = io.BytesIO()
    torch.save(ob.state_dict(), buf)
    buf.seek(0)
    log("resume after 3 steps from torch.save(state_dict())")
    oc = TurboAdam(groups(pb), **KW)  # default seed: the checkpoint restores 31337
    with torch.serialization.safe_globals([CoStateManager]):
        oc.load_state_dict(torch.load(buf, weights_only=True))
    assert oc.philox_seed == 31337
    run(oc, pb, range(3, 5))
    bad = []
    for i, (a, b) in enumerate(zip(pa, pb)):
        if not np.array_equal(_bits(from_torch(a)), _bits(from_torch(b))):
            bad.append(f"tensor {i}: params differ")
        bad += compare_states(gpu_state(oc, b), gpu_state(oa, a), f"tensor {i}")
    assert not bad, "\n".join(bad[:20])
