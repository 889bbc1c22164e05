"""GPU: the reference's public helper functions (turboadam_amd.costate /
quantize / oneq), one tensor per call, against the CPU oracle's functions on
identical inputs.  Bar: bit-exact for every output (indices, scales, signs,
labels, norms, amplitudes, alpha, thresholds, m, v)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import log

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SQRT128 = float(np.float32(np.sqrt(128.0)))


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _np(t):
    t = t.detach().cpu()
    if t.dtype == torch.float16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _same(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), b.view(np.uint32)
    return a.shape == b.shape and np.array_equal(a, b)


def _mg(n, seed):
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    m = (0.4 * g + rng.standard_normal(n).astype(np.float32) * 1e-4).astype(np.float32)
    return m, g


@pytest.mark.parametrize("n", [1, 127, 128, 5000, 70_001, 1_100_000])
def test_decompose_ratios_encode(n):
    from turboadam_amd import costate as C

    log(f"decompose / ratios / encode n={n}")
    m, g = _mg(n, n)
    L = O.lib()
    delta_o = np.empty(n, np.float32)
    alpha_o = L.or_decompose(O.ptr(m), O.ptr(g), n, O.ptr(delta_o))
    alpha, delta = C.decompose(_t(m), _t(g))
    assert _same(np.float32(alpha.item()), np.float32(alpha_o))
    assert _same(_np(delta), delta_o)
    nb = (n + 127) // 128
    ratios_o = np.empty(nb, np.float32)
    L.or_block_ratios(O.ptr(delta_o), O.ptr(m), n, O.ptr(ratios_o))
    ratios = C.compute_block_ratios(delta, _t(m))
    assert _same(_np(ratios), ratios_o)
    signs_o = np.empty((n + 7) // 8, np.uint8)
    norms_o = np.empty(nb, np.float32)
    amp_o = np.empty(nb, np.uint16)
    L.or_encode(O.ptr(delta_o), n, SQRT128, O.ptr(signs_o), O.ptr(norms_o), O.ptr(amp_o))
    labels = torch.zeros(nb, dtype=torch.uint8, device=DEV)
    enc = C.encode_blocks(delta, labels)
    assert _same(_np(enc["sign_packed"]), signs_o)
    assert _same(_np(enc["block_norms"]), norms_o)
    assert _same(_np(enc["scales"]), amp_o)
    assert enc["labels"] is labels


@pytest.mark.parametrize("nb,null_pct,amp_pct", [(1, 0.1, 0.9), (40, 0.1, 0.9), (9000, 0.05, 0.95),
                                                 (40_000, 0.1, 0.9)])
def test_thresholds_and_classify(nb, null_pct, amp_pct):
    from turboadam_amd import costate as C

    log(f"thresholds / classify nb={nb}")
    rng = np.random.default_rng(nb)
    r = np.abs(rng.standard_normal(nb)).astype(np.float32)
    r[rng.integers(0, nb, max(1, nb // 50))] = 0.0          # ties at zero
    r[rng.integers(0, nb, max(1, nb // 50))] = r[0]          # repeated values
    t0o, t1o = np.zeros(1, np.float32), np.zeros(1, np.float32)
    k_lo, k_hi = O.ranks(nb, null_pct, amp_pct)
    O.lib().or_thresholds(O.ptr(r), nb, k_lo, k_hi, O.ptr(t0o), O.ptr(t1o))
    t0, t1 = C.compute_thresholds(_t(r), null_pct, amp_pct)
    assert _same(np.float32(t0.item()), t0o[0]) and _same(np.float32(t1.item()), t1o[0])
    lab_o = np.empty(nb, np.uint8)
    O.lib().or_classify(O.ptr(r), nb, float(t0o[0]), float(t1o[0]), O.ptr(lab_o))
    assert _same(_np(C.classify_blocks(_t(r), t0, t1)), lab_o)
    assert _same(_np(C.classify_blocks(_t(r), float(t0o[0]), float(t1o[0]))), lab_o)


def _edge_ratios(case):
    """Ratio arrays that drive the radix selection through its edge cases."""
    rng = np.random.default_rng(7)
    if case == "all_equal":          # kmin == kmax: no round runs
        return np.full(20_000, 0.37, np.float32)
    if case == "all_zero":
        return np.zeros(8192, np.float32)
    if case == "low_bits":           # keys differ only in their last bits: every round narrows
        return (np.float32(1.0).view(np.uint32) + rng.integers(0, 7, 30_000, dtype=np.uint32)).view(np.float32)
    if case == "two_values":         # one jump between the two ranks
        r = np.full(16_384, 0.5, np.float32)
        r[8000:] = 0.75
        return r
    if case == "nan_and_zero":       # NaN orders last, +0 first
        r = np.abs(rng.standard_normal(8193)).astype(np.float32)
        r[rng.integers(0, 8193, 400)] = np.nan
        r[rng.integers(0, 8193, 400)] = 0.0
        return r
    if case == "nan_at_rank":        # the upper rank lands among the NaNs
        r = np.abs(rng.standard_normal(12_000)).astype(np.float32)
        r[:2400] = np.nan
        return r
    if case == "slice_edge":         # exactly one full slice (8193 keys: nan_and_zero)
        return np.abs(rng.standard_normal(8192)).astype(np.float32)
    raise ValueError(case)


@pytest.mark.parametrize("case", ["all_equal", "all_zero", "low_bits", "two_values", "nan_and_zero", "nan_at_rank",
                                  "slice_edge"])
def test_thresholds_edge_cases(case):
    from turboadam_amd import costate as C

    log(f"thresholds edge case {case}")
    r = _edge_ratios(case)
    nb = r.size
    for null_pct, amp_pct in ((0.1, 0.9), (0.05, 0.95)):
        t0o, t1o = np.zeros(1, np.float32), np.zeros(1, np.float32)
        k_lo, k_hi = O.ranks(nb, null_pct, amp_pct)
        O.lib().or_thresholds(O.ptr(r), nb, k_lo, k_hi, O.ptr(t0o), O.ptr(t1o))
        t0, t1 = C.compute_thresholds(_t(r), null_pct, amp_pct)
        # the oracle's order statistics are plain sorts of the bit patterns
        keys = np.sort(r.view(np.uint32))
        assert t0o.view(np.uint32)[0] == keys[k_lo] and t1o.view(np.uint32)[0] == keys[k_hi]
        assert _same(np.float32(t0.item()), t0o[0]) and _same(np.float32(t1.item()), t1o[0])
        lab_o = np.empty(nb, np.uint8)
        O.lib().or_classify(O.ptr(r), nb, float(t0o[0]), float(t1o[0]), O.ptr(lab_o))
        assert _same(_np(C.classify_blocks(_t(r), t0, t1)), lab_o)


@pytest.mark.parametrize("n", [300, 5000, 70_001])
def test_decode_blocks(n):
    from turboadam_amd import costate as C

    log(f"decode_blocks n={n}")
    rng = np.random.default_rng(n + 1)
    nb = (n + 127) // 128
    labels = rng.integers(0, 3, nb).astype(np.uint8)
    signs = rng.integers(0, 256, (n + 7) // 8).astype(np.uint8)
    norms = np.abs(rng.standard_normal(nb)).astype(np.float32) * 1e-3
    amp = (np.abs(rng.standard_normal(nb)) * 1e-4).astype(np.float16).view(np.uint16)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    alpha = np.float32(0.37)
    want = np.empty(n, np.float32)
    O.lib().or_decode_blocks(O.ptr(labels), O.ptr(signs), O.ptr(norms), O.ptr(amp), float(alpha), O.ptr(g), n,
                             SQRT128, O.ptr(want))
    enc = {"labels": _t(labels), "sign_packed": _t(signs), "block_norms": _t(norms),
           "scales": _t(amp.view(np.float16))}
    got = C.decode_blocks(enc, torch.tensor(alpha, device=DEV), _t(g))
    assert _same(_np(got), want)
    got2 = C.decode_blocks(enc, float(alpha), _t(g))
    assert _same(_np(got2), want)


@pytest.mark.parametrize("null_pct,amp_pct", [(0.10, 0.90), (0.05, 0.95)])
def test_costate_manager_update_steps(null_pct, amp_pct):
    from turboadam_amd import costate as C

    n = 70_001
    log(f"CoStateManager.update n={n}, 5 steps")
    rng = np.random.default_rng(7)
    nb = (n + 127) // 128
    labels = np.zeros(nb, np.uint8)
    signs = np.zeros((n + 7) // 8, np.uint8)
    norms = np.zeros(nb, np.float32)
    amp = np.zeros(nb, np.uint16)
    alpha = np.zeros(1, np.float32)
    mgr = C.CoStateManager(null_pct=null_pct, amp_pct=amp_pct)
    drift = rng.standard_normal(n).astype(np.float32)
    k_lo, k_hi = O.ranks(nb, null_pct, amp_pct)
    for s in range(5):
        g = ((rng.standard_normal(n).astype(np.float32) + 0.3 * drift) * 1e-3).astype(np.float32)
        m_o = np.empty(n, np.float32)
        O.lib().or_costate_update(O.ptr(g), n, O.f32(0.9), O.f32(1.0 - 0.9), SQRT128, k_lo, k_hi, int(s > 0),
                                  O.ptr(labels), O.ptr(signs), O.ptr(norms), O.ptr(amp), O.ptr(alpha), O.ptr(m_o))
        m = mgr.update(_t(g), 0.9)
        enc = mgr._encoded
        assert _same(_np(m), m_o), f"step {s}: m"
        assert _same(_np(enc["labels"]), labels), f"step {s}: labels"
        assert _same(_np(enc["sign_packed"]), signs), f"step {s}: signs"
        assert _same(_np(enc["block_norms"]), norms), f"step {s}: norms"
        assert _same(_np(enc["scales"]), amp), f"step {s}: amp"
        assert _same(np.float32(mgr._alpha.item()), alpha[0]), f"step {s}: alpha"


def test_costate_manager_update_error_feedback():
    from turboadam_amd import costate as C

    n = 70_001
    log(f"CoStateManager.update with error feedback n={n}, 5 steps")
    rng = np.random.default_rng(8)
    nb = (n + 127) // 128
    labels = np.zeros(nb, np.uint8)
    signs = np.zeros((n + 7) // 8, np.uint8)
    norms = np.zeros(nb, np.float32)
    amp = np.zeros(nb, np.uint16)
    alpha = np.zeros(1, np.float32)
    res = np.zeros(n, np.float32)
    mgr = C.CoStateManager(error_feedback=True)
    k_lo, k_hi = O.ranks(nb, 0.10, 0.90)
    for s in range(5):
        g = (rng.standard_normal(n).astype(np.float32) * 1e-3).astype(np.float32)
        m_o = np.empty(n, np.float32)
        O.lib().or_costate_update_ef(O.ptr(g), n, O.f32(0.9), O.f32(1.0 - 0.9), SQRT128, k_lo, k_hi, int(s > 0),
                                     O.ptr(labels), O.ptr(signs), O.ptr(norms), O.ptr(amp), O.ptr(alpha), 1,
                                     int(s > 0), O.ptr(res), O.ptr(m_o))
        m = mgr.update(_t(g), 0.9)
        enc = mgr._encoded
        assert _same(_np(m), m_o), f"step {s}: m"
        assert _same(_np(enc["labels"]), labels), f"step {s}: labels"
        assert _same(_np(enc["sign_packed"]), signs), f"step {s}: signs"
        assert _same(_np(enc["block_norms"]), norms), f"step {s}: norms"
        assert _same(_np(enc["scales"]), amp), f"step {s}: amp"
        assert _same(np.float32(mgr._alpha.item()), alpha[0]), f"step {s}: alpha"
        assert _same(_np(mgr._ef_residual), res), f"step {s}: residual"


@pytest.mark.parametrize("bits,dt", [(4, torch.float32), (2, torch.bfloat16), (8, torch.float32), (6, torch.float16)])
def test_fused_v_update_standalone(bits, dt):
    from turboadam_amd import quantize as Q

    n = 70_001
    log(f"fused_v_update n={n} bits={bits} {dt}")
    rng = np.random.default_rng(bits)
    nb = (n + 127) // 128
    idx = rng.integers(0, 1 << bits, nb * 128).astype(np.uint8)
    lo = rng.uniform(-25, -15, nb).astype(np.float32)
    sc = np.stack([lo, lo + rng.uniform(0, 6, nb).astype(np.float32)], 1).astype(np.float16).view(np.uint16)
    g_t = (torch.from_numpy(rng.standard_normal(n).astype(np.float32)) * 1e-3).to(dt)
    g32 = g_t.float().numpy()
    idx_o, sc_o = idx.copy(), sc.reshape(-1).copy()
    v_o = np.empty(n, np.float32)
    O.lib().or_fused_v_update(O.ptr(idx_o), O.ptr(sc_o), O.ptr(g32), n, bits, O.f32(0.999), O.f32(1.0 - 0.999),
                              5, 9, 1234, O.ptr(v_o))
    ni, ns, v = Q.fused_v_update(_t(idx), _t(sc.view(np.float16)), g_t.to(DEV), 0.999, bits, tensor_id=5, step=9,
                                 seed=1234)
    assert _same(_np(ni), idx_o)
    assert _same(_np(ns).reshape(-1), sc_o)
    assert _same(_np(v), v_o)


@pytest.mark.parametrize("stochastic", [False, True])
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_logscale(stochastic, bits):
    from turboadam_amd import oneq, quantize as Q

    n = 128 * 300
    log(f"quantize_logscale_nbits bits={bits} stochastic={stochastic}")
    rng = np.random.default_rng(bits + 10 * stochastic)
    v = np.exp(rng.uniform(-40, -5, n)).astype(np.float32)
    v[rng.integers(0, n, 50)] = 0.0                   # clamped to 1e-38
    idx_o = np.empty(n, np.uint8)
    sc_o = np.empty(2 * (n // 128), np.uint16)
    O.lib().or_quantize_logscale(O.ptr(v), n, bits, int(stochastic), 3, 4, 99, O.ptr(idx_o), O.ptr(sc_o))
    idx, sc, nbits = Q.quantize_logscale_nbits(_t(v), bits, stochastic_round=stochastic, tensor_id=3, step=4, seed=99)
    assert nbits == bits
    assert _same(_np(idx), idx_o)
    assert _same(_np(sc).reshape(-1), sc_o)
    # round trip through dequantize / decompress, against the oracle's decode
    dq = Q.dequantize_logscale_nbits(idx, sc, bits, original_numel=n)
    assert _same(_np(dq), O.dequantize(idx_o, sc_o, n, bits))
    comp = {"indices": idx, "scales": sc, "n_bits": bits, "original_shape": torch.Size([n]),
            "original_length": n, "block_size": 128}
    assert _same(_np(oneq.decompress_v(comp)), O.dequantize(idx_o, sc_o, n, bits))


def test_dequantize_and_decompress_against_oracle_and_reference():
    """dequantize_logscale_nbits / decompress_v (tam_v_dequantize) on the
    reference's own quantized states (tests/golden): bit-exact against the
    oracle's or_dequantize, and against the reference's outputs except where
    its exp (MKL) is not correctly rounded, by one ulp there."""
    import json
    import os

    from turboadam_amd import oneq, quantize as Q

    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    z = np.load(os.path.join(here, "golden_dequantize.npz"))
    meta = json.loads(str(z["meta"]))
    for name, c in meta["cases"].items():
        q = np.load(os.path.join(here, f"golden_{name}.npz"))
        idx, sc, bits, nb = q["indices"], q["scales"].reshape(-1), c["bits"], c["nb"]
        log(f"dequantize {name}: {nb} blocks, {bits} bits")
        idx_t, sc_t = _t(idx), _t(sc.view(np.float16)).reshape(nb, 2)
        for n, key in ((nb * 128, "full"), (nb * 128 - meta["trim"], "trim")):
            got = _np(Q.dequantize_logscale_nbits(idx_t, sc_t, bits, original_numel=n))
            assert _same(got, O.dequantize(idx, sc, n, bits)), (name, key)
            ref = z[f"{name}_{key}"]
            diff = got.view(np.int32) != ref.view(np.int32)
            assert diff.mean() <= 0.05 and (np.abs(got.view(np.int32) - ref.view(np.int32))[diff] <= 1).all()
        # the reference returns the first nb*128 values for a larger count (quantize.py:214)
        assert _np(Q.dequantize_logscale_nbits(idx_t, sc_t, bits, original_numel=nb * 128 + 5)).size == nb * 128
        if f"{name}_decompress" in z.files:
            n = 5000
            comp = {"indices": idx_t, "scales": sc_t, "n_bits": bits, "original_shape": torch.Size([n]),
                    "original_length": n, "block_size": 128}
            got = _np(oneq.decompress_v(comp))
            assert _same(got, O.dequantize(idx, sc, n, bits))
            ref = z[f"{name}_decompress"]
            assert (np.abs(got.view(np.int32) - ref.view(np.int32)) <= 1).all()


def test_compress_v_logscale_init_closed_form():
    from turboadam_amd import oneq

    log("compress_v_logscale(full(1e-30)) == init_v_state")
    p = torch.empty(5000, device=DEV)
    comp = oneq.compress_v_logscale(torch.full((5000,), 1e-30, device=DEV), n_bits=4)
    init = oneq.init_v_state(p, 4)
    assert torch.equal(comp["indices"], init["indices"])
    assert torch.equal(comp["scales"].view(torch.int16), init["scales"].view(torch.int16))
    assert comp["original_length"] == 5000 and comp["original_shape"] == p.shape


def test_compress_v_logscale_matches_reference_fixture():
    """compress_v_logscale on a ragged v (5000 elements: the last block is padded
    with max(min(v), 1e-38), formed on the device) equals the reference's own
    output (golden_compress_b4: exact zeros, ~35 e-folds of range)."""
    import os

    from tests.golden import make_golden as MG
    from turboadam_amd import oneq

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_compress_b4.npz"))
    v = z["v"]
    case = MG.Q_CASES["compress_b4"]
    comp = oneq.compress_v_logscale(_t(v), n_bits=case["bits"])
    log(f"compress_v_logscale n={v.size} bits={case['bits']} vs the reference fixture")
    assert _same(_np(comp["indices"]), z["indices"])
    assert _same(_np(comp["scales"]).reshape(-1), z["scales"].reshape(-1))
    assert comp["original_length"] == v.size and comp["original_shape"] == torch.Size([v.size])
