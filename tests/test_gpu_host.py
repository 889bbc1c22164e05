"""Steady steps of the host code (GPU): a step whose parameters with gradients
and whose state are those of the previous step skips the per-parameter walk.
Every transition in and out of that path must leave the results bit-identical
to the oracle: new gradient tensors, reused gradient tensors refilled in place,
a gradient that goes missing and comes back, an lr change, a state dict
loaded mid-run and a group added mid-run."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import compare_with_oracle, from_torch, log, to_bits, to_torch

pytestmark = pytest.mark.gpu

F32, BF16 = O.DT_F32, O.DT_BF16


def test_steady_steps_match_oracle_across_transitions():
    from turboadam_amd import TurboAdam

    dev = torch.device("cuda:0")
    sizes = [5000, 300, 4096 + 77, 9000]
    dts = [F32, F32, BF16, BF16]
    rng = np.random.default_rng(51)
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
    params = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    kw = dict(lr=1e-3, weight_decay=0.05)
    opt = TurboAdam(params[:3], philox_seed=21, **kw)
    oparams = [a.copy() for a in init]
    orc = O.OracleTurboAdam(oparams[:3], dtypes=dts[:3], seed=21, **kw)
    kept = [None] * len(sizes)
    taken = []
    fast_step = opt._fast_step

    def spy():
        r = fast_step()
        taken.append(r)
        return r

    opt._fast_step = spy

    def grads(step):
        return [to_bits((rng.standard_normal(n) * 1e-3 * (1 + step % 3)).astype(np.float32), dt)
                for n, dt in zip(sizes, dts)]

    for step in range(12):
        gs = grads(step)
        n_active = 4 if step >= 9 else 3
        if step == 9:  # a group added mid-run: its parameter gets its own group
            opt.add_param_group({"params": [params[3]], "lr": 5e-4})
            orc.add_param_group({"params": [oparams[3]], "lr": 5e-4}, dtypes=[dts[3]])
        if step == 6:  # an lr schedule step
            for grp in opt.param_groups:
                grp["lr"] = 2e-3
            for grp in orc.param_groups:
                grp["lr"] = 2e-3
        if step == 7:  # the optimizer's own state dict, loaded back mid-run
            opt.load_state_dict(opt.state_dict())
        og = []
        for i in range(n_active):
            if step == 4 and i == 1:  # a gradient that goes missing for one step
                params[i].grad = None
                og.append(None)
                continue
            t = to_torch(gs[i], dts[i], (sizes[i],), dev)
            if step in (2, 3, 10) and kept[i] is not None:
                kept[i].copy_(t)  # the same gradient object, refilled in place
                params[i].grad = kept[i]
            else:
                params[i].grad = kept[i] = t
            og.append(gs[i])
        opt.step()
        orc.step(og)
        torch.cuda.synchronize()
        bad = compare_with_oracle(opt, params[:n_active], orc, oparams[:n_active], f"step {step + 1}")
        assert not bad, "\n".join(bad[:20])
    log(f"12 steps; steady path taken at steps {[i + 1 for i, r in enumerate(taken) if r]}")
    assert sum(taken) >= 5
    assert taken[-1]  # the last step was steady again


def test_replaced_parameter_storage_is_followed():
    """A parameter whose storage is replaced between steps (p.data = a copy,
    then p.data = p.data.to(bf16)) is stepped in its new storage and dtype, on
    the steady path's terms: the descriptor rows follow the parameter, not the
    storage they were built on.  The old storages stay referenced, so a stale
    row would update them instead and show as a mismatch."""
    from turboadam_amd import TurboAdam

    dev = torch.device("cuda:0")
    sizes = [5000, 4096 + 77, 300]
    dts = [F32, F32, BF16]
    rng = np.random.default_rng(52)
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
    params = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    kw = dict(lr=1e-3, weight_decay=0.01)
    opt = TurboAdam(params, philox_seed=22, **kw)
    oparams = [a.copy() for a in init]
    orc = O.OracleTurboAdam(oparams, dtypes=list(dts), seed=22, **kw)
    old = []
    for step in range(8):
        if step == 3:  # same values, new storage
            old.append(params[0].data)
            params[0].data = params[0].data.clone()
        if step == 5:  # fp32 -> bf16 (round to nearest even, as the oracle's copy)
            old.append(params[1].data)
            params[1].data = params[1].data.to(torch.bfloat16)
            dts[1] = BF16
            oparams[1] = to_bits(oparams[1], BF16)
            orc.param_groups[0]["params"][1] = oparams[1]
            orc.dtypes[1] = BF16
        gs = [to_bits((rng.standard_normal(n) * 1e-3).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
        for p, g, dt, n in zip(params, gs, dts, sizes):
            p.grad = to_torch(g, dt, (n,), dev)
        opt.step()
        orc.step(gs)
        torch.cuda.synchronize()
        bad = compare_with_oracle(opt, params, orc, oparams, f"step {step + 1}")
        assert not bad, "\n".join(bad[:20])
    assert params[1].dtype == torch.bfloat16
    log("8 steps with a storage swap at step 4 and an fp32 -> bf16 swap at step 6")


def test_replaced_or_reset_state_is_followed():
    """State tensors replaced between steps by copies of themselves (exp_avg,
    the 1Q indices and scales, every CoState array and alpha), and state
    reset by opt.state[p] = {} and by opt.state.clear(): each following step
    must step the state that opt.state now holds, re-initialised where it was
    reset, as the oracle does.  The replaced tensors stay referenced, so a
    descriptor row that kept pointing at them would update them instead and
    show as a mismatch.  Gradients are new tensors every step, so every other
    step takes the steady path."""
    from turboadam_amd import TurboAdam

    dev = torch.device("cuda:0")
    sizes = [5000, 300, 4096 + 77, 9000]
    dts = [F32, F32, BF16, BF16]
    rng = np.random.default_rng(53)
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
    params = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    kw = dict(lr=1e-3, weight_decay=0.02)
    opt = TurboAdam(params, philox_seed=23, **kw)
    oparams = [a.copy() for a in init]
    orc = O.OracleTurboAdam(oparams, dtypes=list(dts), seed=23, **kw)
    taken = []
    fast_step = opt._fast_step

    def spy():
        r = fast_step()
        taken.append(r)
        return r

    opt._fast_step = spy
    old = []  # replaced tensors, kept alive

    def swap(holder, key):
        old.append(holder[key])
        holder[key] = holder[key].clone()

    for step in range(14):
        if step == 3:  # same values, new tensors
            st0, st1 = opt.state[params[0]], opt.state[params[1]]
            swap(st1, "exp_avg")
            swap(st0["compressed_v"], "indices")
            swap(st1["compressed_v"], "scales")
            enc = st0["m_mgr"]._encoded
            for key in ("sign_packed", "labels", "block_norms", "scales"):
                swap(enc, key)
        if step == 5:
            mgr = opt.state[params[2]]["m_mgr"]
            old.append(mgr._alpha)
            mgr._alpha = mgr._alpha.clone()
        if step == 7:  # one parameter's state reset: initialised again at this step
            opt.state[params[2]] = {}
            del orc.state[2]
        if step == 10:  # every state reset
            opt.state.clear()
            orc.state.clear()
        gs = [to_bits((rng.standard_normal(n) * 1e-3 * (1 + step % 3)).astype(np.float32), dt)
              for n, dt in zip(sizes, dts)]
        for p, g, dt, n in zip(params, gs, dts, sizes):
            p.grad = to_torch(g, dt, (n,), dev)
        opt.step()
        orc.step(gs)
        torch.cuda.synchronize()
        bad = compare_with_oracle(opt, params, orc, oparams, f"step {step + 1}")
        assert not bad, "\n".join(bad[:20])
    steady = [i + 1 for i, r in enumerate(taken) if r]
    log(f"14 steps; steady path taken at steps {steady}")
    for s in (4, 6, 8, 11):  # the step after each change takes the full path
        assert s not in steady
    assert taken[-1]
