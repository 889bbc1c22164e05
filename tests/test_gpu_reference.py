"""GPU against the reference's own outputs (tests/golden fixtures), end to end.

The fixtures hold what the reference CPU path produced for inputs that
oracle/inputs.py regenerates, with this build's Philox draws injected.  The
GPU step (through the C ABI) runs on the same inputs and draws.  Bars (from the
parity targets): parameters within 1e-6 relative (norm-wise per tensor) after
short runs and within 1e-4 over the 200-step trajectory; 1Q indices may
differ only on ties of the reference's library arithmetic (MKL exp / log vs
the correctly rounded definitions), so at most a tiny fraction of them.
CoState sign bits and labels are not compared end to end: at step 1,
m = fl(0.1 g) and alpha ~ 0.1, so delta = m - alpha*g is rounding noise whose
signs follow alpha's last bit (MKL's dot vs the exact one), and later steps
carry those signs forward.  tests/test_golden.py checks them one step at a
time from a common state instead (each difference within its tie margin)."""

import json
import os
import sys

import numpy as np
import pytest
import torch

from tests.helpers import from_torch, gpu_state, log

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as MG  # noqa: E402

pytestmark = pytest.mark.gpu

SHORT = [c for c in MG.CASES if c not in ("traj_f32", "gpt2_block")]


def _run(name, on_step=None):
    from turboadam_amd import TurboAdam

    case = MG.CASES[name]
    dev = torch.device("cuda:0")
    init, sig = MG.case_inputs(case)
    shapes = case.get("shapes") or [(n,) for n in case["sizes"]]
    params = [torch.nn.Parameter(MG.from_bits(a, case["dt"]).reshape(s).to(dev)) for a, s in zip(init, shapes)]
    opt = TurboAdam(params, **case["kw"])
    opt.philox_seed = MG.SR_SEED
    for s in range(case["steps"]):
        for p, g, shp in zip(params, MG.step_grads(case, sig, s), shapes):
            p.grad = MG.from_bits(g, case["dt"]).reshape(shp).to(dev)
        opt.step()
        if on_step is not None:
            on_step(s + 1, opt, params)
    torch.cuda.synchronize()
    return case, opt, params


def _as_f32(a, dt):
    if dt == 0:
        return a.astype(np.float64)
    return MG.from_bits(a, dt).float().numpy().astype(np.float64)


def _rel(a, b):
    d = np.linalg.norm(a - b)
    s = np.linalg.norm(b)
    return d / s if s > 0 else d


def _ulp16_flips(a, b):
    """Elements of two 16-bit parameter arrays (bit patterns) that differ, and
    whether each differs by one unit in the last place only (neighbouring
    patterns of one sign)."""
    a16, b16 = a.astype(np.int32), b.astype(np.int32)
    diff = a16 != b16
    one_ulp = (np.abs(a16 - b16) == 1) & ((a16 & 0x8000) == (b16 & 0x8000))
    return int(diff.sum()), bool(one_ulp[diff].all())


@pytest.mark.parametrize("name", SHORT)
def test_gpu_matches_reference_fixtures(name):
    log(f"GPU vs reference fixture {name}")
    z = np.load(os.path.join(HERE, "golden", f"golden_{name}.npz"))
    case, opt, params = _run(name)
    dt = case["dt"]
    frac_bad = []
    # With error feedback a sign bit that flips at a tie (|delta| within the
    # alpha difference) moves that element's residual by a whole block scale,
    # which the following steps' m carry: the CPU restatement in exact mode
    # (which the GPU equals bit for bit) ends 4.7e-5 from the reference on
    # ef_f32 (tests/test_golden.py::test_error_feedback_end_to_end_ties).
    # End to end, a 16-bit parameter can also land one unit in the last place
    # off: CoState's first-step sign bits follow alpha's last bit (see above),
    # so m differs by rounding noise from the first step on, and now and then
    # an update sits on a 16-bit rounding boundary.  One such element of a
    # small tensor exceeds 1e-6 norm-wise (one fp16 ulp of 8192 elements is
    # 4e-6); each step from a common state stays within 1e-6
    # (tests/test_golden.py::test_exact_and_faithful_differ_only_by_ties).
    tol = 1e-4 if case["kw"].get("error_feedback") else 1e-6
    for i, p in enumerate(params):
        got, want = from_torch(p.data), z[f"param_{i}"]
        pr = _rel(_as_f32(got, dt), _as_f32(want, dt))
        if pr > tol and dt != 0:
            nd, one_ulp = _ulp16_flips(got, want)
            assert one_ulp and nd <= max(2, 1e-3 * got.size), \
                f"{name} tensor {i}: param rel {pr:.3g}, {nd} elements differ (one ulp each: {one_ulp})"
            log(f"{name} tensor {i}: {nd} element(s) one 16-bit ulp off the reference (rel {pr:.3g})")
        else:
            assert pr <= tol, f"{name} tensor {i}: param rel {pr:.3g}"
        st = gpu_state(opt, p)
        for k in ("indices",):
            if f"{k}_{i}" in z.files:
                a, b = st[k], z[f"{k}_{i}"]
                assert a.shape == b.shape
                frac_bad.append(np.count_nonzero(a != b) / max(1, a.size))
    assert max(frac_bad, default=0.0) <= 1e-3, f"{name}: 1Q index mismatch fraction {max(frac_bad):.3g}"


def test_gpu_gpt2_block_matches_reference_samples():
    """The GPT-2-small block (12 fp32 tensors, 7.1M params, 3 steps): the
    reference fixture keeps every 997th element of each final parameter
    (golden_gpt2_block psample_*); the GPU's are within 1e-6 norm-wise.  The
    fixture's per-step digests cover the CoState sign bits, which differ at
    the ties described above; tests/test_golden.py checks them on the CPU."""
    log("GPU vs reference fixture gpt2_block (sampled parameters)")
    z = np.load(os.path.join(HERE, "golden", "golden_gpt2_block.npz"))
    meta = json.loads(str(z["meta"]))
    case, opt, params = _run("gpt2_block")
    assert meta["steps"] == case["steps"]
    for i, p in enumerate(params):
        got = from_torch(p.data)[::997].astype(np.float64)
        want = z[f"psample_{i}"].astype(np.float64)
        assert got.shape == want.shape
        pr = _rel(got, want)
        assert pr <= 1e-6, f"gpt2_block tensor {i}: sampled param rel {pr:.3g}"


def test_gpu_200_step_trajectory_matches_reference():
    log("GPU vs reference 200-step trajectory (traj_f32)")
    z = np.load(os.path.join(HERE, "golden", "golden_traj_f32.npz"))
    meta = json.loads(str(z["meta"]))
    worst = {}

    def check(step, opt, params):
        if step in meta["keep_params"]:
            torch.cuda.synchronize()
            for i, p in enumerate(params):
                r = _rel(from_torch(p.data).astype(np.float64), z[f"p{step}_{i}"].astype(np.float64))
                worst[(step, i)] = r

    _run("traj_f32", check)
    assert worst and max(worst.values()) <= 1e-4, worst


def test_gpu_groups_none_gradients_and_add_param_group():
    """Two groups with their own hyperparameters, None gradients (a late
    parameter that sets its group's shared bias corrections, a parameter
    skipped after its first step) and a group added before step 5: the GPU
    equals the oracle bit for bit every step, and ends within 1e-6 of the
    reference's parameters (tests/golden/golden_groups.npz) with its step counts."""
    from oracle import oracle as O
    from tests.helpers import compare_states
    from turboadam_amd import TurboAdam

    log("GPU vs oracle and reference: param groups, None gradients, add_param_group")
    z = np.load(os.path.join(HERE, "golden", "golden_groups.npz"))
    case = MG.GROUPS_CASE
    dev = torch.device("cuda:0")
    init, sig = MG.case_inputs(case)
    params = [torch.nn.Parameter(MG.from_bits(a, case["dt"]).to(dev)) for a in init]
    opt = TurboAdam([{"params": [params[i] for i in g["idx"]], **g["kw"]} for g in case["groups"]],
                    philox_seed=MG.SR_SEED, **case["kw"])
    oparams = [a.copy() for a in init]
    orc = O.OracleTurboAdam([{"params": [oparams[i] for i in g["idx"]], **g["kw"]} for g in case["groups"]],
                            dtypes=[case["dt"]] * 4, seed=MG.SR_SEED, **case["kw"])
    bad = []
    for s in range(case["steps"]):
        if s == case["added"]["before_step"]:
            added = case["added"]
            opt.add_param_group({"params": [params[i] for i in added["idx"]], **added["kw"]})
            orc.add_param_group({"params": [oparams[i] for i in added["idx"]], **added["kw"]}, dtypes=[case["dt"]])
        grads = MG.groups_grads(case, sig, s)
        for p, g in zip(params, grads):
            p.grad = None if g is None else MG.from_bits(g, case["dt"]).to(dev)
        opt.step()
        orc.step(grads)
        torch.cuda.synchronize()
        for i, p in enumerate(params):
            if not np.array_equal(from_torch(p.data).view(np.uint32), oparams[i].view(np.uint32)):
                bad.append(f"step {s + 1} tensor {i}: params differ")
            if i in orc.state:
                bad += compare_states(gpu_state(opt, p), orc.state[i], f"step {s + 1} tensor {i}")
    assert not bad, "\n".join(bad[:20])
    for i, p in enumerate(params):
        pr = _rel(from_torch(p.data).astype(np.float64), z[f"param_{i}"].astype(np.float64))
        assert pr <= 1e-6, f"tensor {i}: param rel {pr:.3g}"
        assert opt.state[p]["step"] == int(z[f"step_{i}"])
