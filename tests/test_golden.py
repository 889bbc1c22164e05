"""CPU: the oracle against the reference's own outputs (tests/golden fixtures).

The fixtures were written by tests/golden/make_golden.py, which ran the
reference CPU path (davidkny22/turboadam) with the Philox uniforms of this
build injected into its single torch.rand_like call.  Three links:

1. oracle/torch_mirror.py in faithful mode (literal torch ops) reproduces the
   reference's per-step parameters and packed state bit for bit;
2. the mirror in exact mode (the five library-defined operations replaced by
   their exact definitions) equals the C oracle bit for bit;
3. one step from the same state in both modes differs only by documented ties:
   each differing sign bit, label, index or scale lies within the margin its
   operation's last-bit difference explains, and alpha / parameters agree to
   the stated relative bounds.
So the C oracle (and the GPU, which equals it) is the reference algorithm with
exactly those operations fixed.
"""

import copy
import hashlib
import json
import os
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import torch_mirror as TM

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as MG  # noqa: E402  (fixture definitions: cases and input generation)

CASES = list(MG.CASES)
FAST = [c for c in CASES if c not in ("traj_f32", "gpt2_block")]


def _load(name):
    z = np.load(os.path.join(HERE, "golden", f"golden_{name}.npz"))
    return z, json.loads(str(z["meta"]))


def _mirror(name, ops):
    case = MG.CASES[name]
    init, sig = MG.case_inputs(case)
    shapes = case.get("shapes") or [(n,) for n in case["sizes"]]
    params = [MG.from_bits(a, case["dt"]).reshape(s) for a, s in zip(init, shapes)]
    opt = TM.MirrorTurboAdam(params, ops=ops, seed=MG.SR_SEED, **case["kw"])
    return case, sig, shapes, params, opt


def _step_grads(case, sig, s, shapes):
    return [MG.from_bits(g, case["dt"]).reshape(sh) for g, sh in zip(MG.step_grads(case, sig, s), shapes)]


def _digest(opt, p, i):
    arrs = opt.arrays(i)
    arrs["param"] = MG.np_of(p)
    return MG.digest(arrs)


@pytest.fixture(autouse=True)
def _one_thread():
    n = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(n)


@pytest.mark.parametrize("name", CASES)
def test_faithful_mirror_reproduces_reference(name):
    z, meta = _load(name)
    case, sig, shapes, params, opt = _mirror(name, TM.FaithfulOps)
    for s in range(case["steps"]):
        opt.step(_step_grads(case, sig, s, shapes))
        got = [_digest(opt, p, i) for i, p in enumerate(params)]
        assert got == meta["digests"][s], f"{name}: step {s + 1} differs from the reference"


@pytest.mark.parametrize("name", FAST + ["traj_f32"])
def test_exact_mirror_equals_c_oracle(name):
    case, sig, shapes, params, opt = _mirror(name, TM.ExactOps)
    init, _ = MG.case_inputs(case)
    oparams = [a.copy() for a in init]
    orc = O.OracleTurboAdam(oparams, dtypes=[case["dt"]] * len(oparams), seed=MG.SR_SEED, **case["kw"])
    for s in range(case["steps"]):
        opt.step(_step_grads(case, sig, s, shapes))
        orc.step(MG.step_grads(case, sig, s))
        for i, p in enumerate(params):
            a = opt.arrays(i)
            b = orc.state[i]
            assert np.array_equal(MG.np_of(p), oparams[i]), f"{name} step {s + 1} param {i}"
            for k, v in a.items():
                assert np.array_equal(v, b[k]), f"{name} step {s + 1} tensor {i} {k}"


def _ties(case, sig, shapes, params, opt, s):
    """One step from the same state in both modes; returns tie statistics or raises."""
    grads = _step_grads(case, sig, s, shapes)
    pf = [p.clone() for p in params]
    pe = [p.clone() for p in params]
    of = copy.deepcopy(opt)
    oe = copy.deepcopy(opt)
    of.params, oe.params = pf, pe
    tf, te = {}, {}
    of.step(grads, ops=TM.FaithfulOps, traces=tf)
    oe.step(grads, ops=TM.ExactOps, traces=te)
    stats = dict(sign=0, label=0, index=0, scale=0, amp=0, alpha_rel=0.0, param_rel=0.0)
    for i in range(len(params)):
        a, b = of.arrays(i), oe.arrays(i)
        f, e = tf[i], te[i]
        if "alpha" in a and "m" in f:
            al_f, al_e = float(f["alpha"]), float(e["alpha"])
            mg_abs = float((f["m"].double().abs() * grads[i].reshape(-1).double().abs()).sum())
            gg = float((grads[i].reshape(-1).double() ** 2).sum())
            scale = abs(al_f) + (mg_abs / gg if gg > 0 else 0.0)
            d_al = abs(al_f - al_e)
            assert d_al <= 2.0**-19 * scale, f"alpha {al_f} vs {al_e}"
            stats["alpha_rel"] = max(stats["alpha_rel"], d_al / max(abs(al_f), 1e-30))
            # sign bits: a flip needs |delta_i| within what the alpha difference moves it
            g = grads[i].reshape(-1).float()
            df, de = f["delta"], e["delta"]
            flip = (df < 0) != (de < 0)
            tol = d_al * g.abs() + 2.0**-22 * (f["m"].abs() + (f["alpha"] * g).abs())
            assert bool((df[flip].abs() <= tol[flip]).all()), "sign flip outside its margin"
            stats["sign"] += int(flip.sum())
            # labels: a change needs the ratio near a threshold
            rf, re = f["ratios"], e["ratios"]
            lab = a["labels"] != b["labels"]
            if lab.any():
                t0f, t1f = (float(t) for t in f["tau"])
                t0e, t1e = (float(t) for t in e["tau"])
                rel = (rf - re).abs() / rf.abs().clamp(min=1e-30)
                margin = 2.0**-18 + float(rel.max())
                for bi in np.flatnonzero(lab):
                    r1, r2 = float(rf[bi]), float(re[bi])
                    near = min(abs(r1 - t) / max(abs(t), 1e-30) for t in (t0f, t1f, t0e, t1e))
                    near2 = min(abs(r2 - t) / max(abs(t), 1e-30) for t in (t0f, t1f, t0e, t1e))
                    assert min(near, near2) <= margin + abs(t0f - t0e) / max(abs(t0f), 1e-30) + \
                        abs(t1f - t1e) / max(abs(t1f), 1e-30), "label change away from a threshold"
                stats["label"] += int(lab.sum())
            nf, ne = a["block_norms"], b["block_norms"]
            dd = (f["delta"] - e["delta"]).double()
            dpad = torch.cat([dd, dd.new_zeros((-dd.numel()) % 128)]).reshape(-1, 128).norm(dim=1).numpy()
            ok = np.abs(nf.astype(np.float64) - ne) <= 2.0**-20 * np.maximum(np.abs(nf), np.abs(ne)) + dpad + 1e-38
            assert ok.all(), "block norm differs beyond its delta difference"
            stats["amp"] += int(np.count_nonzero(a["amp"] != b["amp"]))
        if "indices" in a:
            cf, ce, u = f["c"], e["c"], f["u"]
            diff = a["indices"] != b["indices"]
            if diff.any():
                d = (cf - u).reshape(-1)[torch.from_numpy(diff)]
                dist = (d - d.round()).abs()
                dc = (cf - ce).abs().reshape(-1)[torch.from_numpy(diff)]
                assert bool((dist <= dc + 1e-6).all()), "index change away from a rounding boundary"
                stats["index"] += int(diff.sum())
            stats["scale"] += int(np.count_nonzero(a["scales"] != b["scales"]))
        x, y = pf[i].double().reshape(-1), pe[i].double().reshape(-1)
        rel = float((x - y).norm() / x.norm().clamp(min=1e-30))  # ||dp||_2 / ||p||_2 per tensor
        stats["param_rel"] = max(stats["param_rel"], rel)
    return stats


@pytest.mark.parametrize("name", FAST + ["traj_f32"])
def test_exact_and_faithful_differ_only_by_ties(name):
    case, sig, shapes, params, opt = _mirror(name, TM.FaithfulOps)
    total = {}
    steps = min(case["steps"], 12)
    for s in range(steps):
        st = _ties(case, sig, shapes, params, opt, s)
        for k, v in st.items():
            total[k] = max(total.get(k, 0), v) if isinstance(v, float) else total.get(k, 0) + v
        opt.step(_step_grads(case, sig, s, shapes))
    print(name, json.dumps(total))
    # alpha within 1e-6 relative of the reference's (MKL sdot) every step
    assert total["alpha_rel"] <= 1e-6
    # parameters move by at most a few ulps per step (sqrt and division inputs agree to the last bit or two)
    assert total["param_rel"] <= 1e-6


@pytest.mark.parametrize("name", list(MG.Q_CASES))
def test_oracle_quantizer_matches_reference(name):
    """or_quantize_logscale (and the compress_v_logscale padding) against the
    reference's quantize_logscale_nbits / compress_v_logscale outputs, including
    the stochastic branch fed the same Philox draws."""
    case = MG.Q_CASES[name]
    z = np.load(os.path.join(HERE, "golden", f"golden_{name}.npz"))
    v = z["v"]
    if case["fn"] == "compress":  # oneq.py:31-34: pad with max(min(v), 1e-38)
        n = v.size
        npad = (n + 127) // 128 * 128
        v = np.concatenate([v, np.full(npad - n, np.float32(max(float(v.min()), 1e-38)), np.float32)])
    npad = v.size
    idx = np.empty(npad, np.uint8)
    sc = np.empty(2 * (npad // 128), np.uint16)
    O.lib().or_quantize_logscale(O.ptr(v), npad, case["bits"], int(case["stochastic"]), case.get("tid", 0),
                                 case.get("step", 1), MG.SR_SEED, O.ptr(idx), O.ptr(sc))
    assert np.array_equal(idx, z["indices"])
    assert np.array_equal(sc, z["scales"].reshape(-1))


@pytest.mark.parametrize("name", [c for c in CASES if MG.CASES[c]["kw"].get("error_feedback")])
def test_error_feedback_end_to_end_ties(name):
    """With error feedback, tie differences (sign bits flipped where |delta| is
    within the alpha difference) enter the residual at a whole block scale and
    stay in m; exact mode therefore ends further from the reference than
    without it, still within 1e-4 in parameters (4.7e-5 on ef_f32), while
    every single step from a common state differs only by ties
    (test_exact_and_faithful_differ_only_by_ties)."""
    case = MG.CASES[name]
    init, sig = MG.case_inputs(case)
    shapes = case.get("shapes") or [(n,) for n in case["sizes"]]
    out = {}
    for mode, ops in (("faithful", TM.FaithfulOps), ("exact", TM.ExactOps)):
        _, _, _, params, opt = _mirror(name, ops)
        for s in range(case["steps"]):
            opt.step(_step_grads(case, sig, s, shapes))
        out[mode] = [p.double().reshape(-1) for p in params]
    for i, (a, b) in enumerate(zip(out["exact"], out["faithful"])):
        rel = float((a - b).norm() / b.norm())
        assert rel <= 1e-4, f"{name} tensor {i}: {rel:.3g}"


def test_oracle_dequantize_matches_reference_and_exact_exp():
    """or_dequantize (the 1Q decode of dequantize_logscale_nbits / decompress_v,
    quantize.py:183-214, oneq.py:51-67) on the reference's own quantized
    states: equal to the reference's outputs except where its exp (MKL) is
    not correctly rounded -- one ulp, on a small fraction -- and equal, bit for
    bit, to exp evaluated in 50-digit decimal and rounded once, of the
    reference's fp32 argument lmin + ((idx + 0.5) / 2^bits) * span."""
    import decimal

    decimal.getcontext().prec = 50
    z = np.load(os.path.join(HERE, "golden", "golden_dequantize.npz"))
    meta = json.loads(str(z["meta"]))
    rng = np.random.default_rng(9)
    for name, c in meta["cases"].items():
        q = np.load(os.path.join(HERE, "golden", f"golden_{name}.npz"))
        idx, sc, bits, nb = q["indices"], q["scales"].reshape(-1), c["bits"], c["nb"]
        full = O.dequantize(idx, sc, nb * 128, bits)
        ref = z[f"{name}_full"]
        diff = full.view(np.int32) != ref.view(np.int32)
        assert diff.mean() <= 0.05, (name, diff.mean())  # MKL exp: within 1 ulp, not always correctly rounded
        assert (np.abs(full.view(np.int32) - ref.view(np.int32))[diff] <= 1).all()
        n = nb * 128 - meta["trim"]
        assert np.array_equal(O.dequantize(idx, sc, n, bits), full[:n])
        assert z[f"{name}_trim"].size == n
        if f"{name}_decompress" in z.files:
            assert np.array_equal(O.dequantize(idx, sc, 5000, bits).view(np.int32),
                                  full[:5000].view(np.int32))
            assert (np.abs(full[:5000].view(np.int32) - z[f"{name}_decompress"].view(np.int32)) <= 1).all()
        # the oracle against exact decimal exp of the same fp32 argument
        lmin = sc[0::2].view(np.float16).astype(np.float32)
        span = (sc[1::2].view(np.float16).astype(np.float32) - lmin).astype(np.float32)
        for i in rng.integers(0, nb * 128, 300):
            b = i // 128
            t = np.float32(np.float32(idx[i]) + np.float32(0.5)) / np.float32(2 ** bits)
            lv = np.float32(lmin[b] + np.float32(t * span[b]))
            y = decimal.Decimal(float(lv)).exp()
            f = np.float32(float(y))
            cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
            want = min(cands, key=lambda v: (abs(decimal.Decimal(float(v)) - y), int(np.float32(v).view(np.uint32)) & 1))
            assert full[i].view(np.uint32) == np.float32(want).view(np.uint32), (name, int(i))


# ---------------------------------------------------------------- host logic: groups, None gradients, add_param_group
def _groups_mirror(ops):
    case = MG.GROUPS_CASE
    init, sig = MG.case_inputs(case)
    params = [MG.from_bits(a, case["dt"]) for a in init]
    opt = TM.MirrorTurboAdam([{"params": [params[i] for i in g["idx"]], **g["kw"]} for g in case["groups"]],
                             ops=ops, seed=MG.SR_SEED, **case["kw"])
    return case, sig, params, opt


def _groups_torch_grads(case, sig, s):
    return [None if g is None else MG.from_bits(g, case["dt"]) for g in MG.groups_grads(case, sig, s)]


def test_faithful_mirror_reproduces_reference_groups():
    """Two groups with their own hyperparameters, None gradients (a late
    parameter that, as its group's last parameter with state, sets the group's
    shared bias corrections; a parameter skipped after its first step) and a
    group added before step 5: the faithful mirror equals the reference's
    per-step digests."""
    z, meta = _load("groups")
    case, sig, params, opt = _groups_mirror(TM.FaithfulOps)
    for s in range(case["steps"]):
        if s == case["added"]["before_step"]:
            opt.add_param_group({"params": [params[i] for i in case["added"]["idx"]], **case["added"]["kw"]})
        opt.step(_groups_torch_grads(case, sig, s))
        got = []
        for i, p in enumerate(params):
            arrs = opt.arrays(i) if i in opt.state else {}
            arrs["param"] = MG.np_of(p)
            got.append(MG.digest(arrs))
        assert got == meta["digests"][s], f"groups: step {s + 1} differs from the reference"
    for i in range(len(params)):
        assert opt.state[i]["step"] == int(z[f"step_{i}"])


def test_exact_mirror_equals_c_oracle_groups():
    case, sig, params, opt = _groups_mirror(TM.ExactOps)
    init, _ = MG.case_inputs(case)
    oparams = [a.copy() for a in init]
    orc = O.OracleTurboAdam([{"params": [oparams[i] for i in g["idx"]], **g["kw"]} for g in case["groups"]],
                            dtypes=[case["dt"]] * 4, seed=MG.SR_SEED, **case["kw"])
    for s in range(case["steps"]):
        if s == case["added"]["before_step"]:
            opt.add_param_group({"params": [params[i] for i in case["added"]["idx"]], **case["added"]["kw"]})
            orc.add_param_group({"params": [oparams[i] for i in case["added"]["idx"]], **case["added"]["kw"]},
                                dtypes=[case["dt"]])
        opt.step(_groups_torch_grads(case, sig, s))
        orc.step(MG.groups_grads(case, sig, s))
        for i, p in enumerate(params):
            assert np.array_equal(MG.np_of(p), oparams[i]), f"step {s + 1} param {i}"
            if i in opt.state:
                for k, v in opt.arrays(i).items():
                    assert np.array_equal(v, orc.state[i][k]), f"step {s + 1} tensor {i} {k}"
