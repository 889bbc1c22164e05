"""Parity at the benchmark configurations' full sizes (GPU, through the C ABI).

A parameter's update depends on that parameter alone: alpha and the two
thresholds are per tensor, and the Philox counter carries the parameter's index.
A full-size step is therefore checked against the oracle tensor by tensor, at
the tensors' real sizes, while the GPU steps the whole configuration in its
fused passes.  Without CoState the blocks of a parameter are independent as
well, so block-aligned slices of a 2^28-element parameter check against the
oracle with their block offset.

Every tensor is also checked for properties that hold at any size:
* the 1Q indices lie below 2^bits;
* each block's fp16 scales are ordered;
* the CoState labels agree with the threshold ranks: at most k_lo blocks fall
  below the k_lo-th smallest ratio, and at least nb - k_hi reach the k_hi-th.
"""

import math

import numpy as np
import pytest
import torch

import bench
from oracle import oracle as O
from tests.helpers import compare_states, compare_with_oracle, f16_bits, from_torch, gpu_state, log

pytestmark = pytest.mark.gpu

SEED = 20251


def _param_bits(t: torch.Tensor) -> np.ndarray:
    a = from_torch(t)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def _invariants(opt, params, v_bits, null_pct=0.10, amp_pct=0.90):
    bad = []
    for i, p in enumerate(params):
        st = opt.state[p]
        nb = (p.numel() + 127) // 128
        cv = st["compressed_v"]
        top = int(cv["indices"].max())
        if top >= (1 << v_bits):
            bad.append(f"tensor {i}: index {top} >= 2^{v_bits}")
        sc = cv["scales"].float().reshape(nb, 2)
        if not bool((sc[:, 0] <= sc[:, 1]).all()):
            bad.append(f"tensor {i}: unordered 1Q scales")
        if st["_compress_m"]:
            k_lo, k_hi = O.ranks(nb, null_pct, amp_pct)
            cnt = torch.bincount(st["m_mgr"]._encoded["labels"].long(), minlength=3).cpu().tolist()
            if len(cnt) != 3 or sum(cnt) != nb or cnt[0] > k_lo or cnt[2] < nb - k_hi:
                bad.append(f"tensor {i}: label counts {cnt} against ranks ({k_lo}, {k_hi}) of {nb} blocks")
    return bad


def _compare_spot(opt, params, orc, spot, where):
    bad = []
    for j, i in enumerate(spot):
        gp = _param_bits(params[i])
        op = orc.param_groups[0]["params"][j]
        op = op.view(np.uint32) if op.dtype == np.float32 else op
        nd = int(np.count_nonzero(gp != op))
        if nd:
            bad.append(f"{where} tensor {i}: params differ in {nd}/{gp.size}")
        bad += compare_states(gpu_state(opt, params[i]), orc.state[j], f"{where} tensor {i}")
    return bad


def test_llama3_8b_shaped_full_steps():
    """Config C3: all 291 bf16 tensors (8.03e9 params) stepped on the GPU for
    its 20 timed steps; both norm shapes, a k and a q projection against the
    oracle at every step, and the 525M-parameter embedding (4.1M blocks: the
    multi-chunk alpha reduction and the multi-slice threshold selection at
    their largest) at steps 1-3."""
    from turboadam_amd import TurboAdam

    shapes = bench.llama3_8b_shapes()
    names = [s[0] for s in shapes]
    spot = [names.index(k) for k in ("l0.norm1", "l0.k", "l31.q", "norm")]
    big = [names.index("embed")]
    steps, big_steps = 20, 3
    log(f"C3 full size: {len(shapes)} tensors, {steps} steps; spot checks {[names[i] for i in spot]} every step, "
        f"{[names[i] for i in big]} at steps 1-{big_steps}")
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    params = []
    for name, shp in shapes:
        p = torch.empty(shp, dtype=torch.bfloat16, device=dev)
        if "norm" in name:
            p.fill_(1.0)
        else:
            p.normal_(0.0, 0.02, generator=gen)
        params.append(torch.nn.Parameter(p))
    kw = dict(lr=3e-4, weight_decay=0.1, v_bits=4)
    opt = TurboAdam(params, philox_seed=SEED, **kw)
    # a parameter's step depends on that parameter alone (and on the step
    # count, equal for all): separate oracles for the two sets
    orc = O.OracleTurboAdam([from_torch(params[i]) for i in spot], dtypes=[O.DT_BF16] * len(spot), seed=SEED,
                            tensor_ids=spot, **kw)
    orc_big = O.OracleTurboAdam([from_torch(params[i]) for i in big], dtypes=[O.DT_BF16] * len(big), seed=SEED,
                                tensor_ids=big, **kw)
    sig = np.exp(math.log(1e-4) + np.random.default_rng(1).standard_normal(len(shapes)))
    bad = []
    for step in range(steps):
        for i, p in enumerate(params):
            g = torch.randn(p.shape, device=dev, generator=gen, dtype=torch.float32)
            p.grad = g.mul_(float(sig[i])).to(torch.bfloat16)
            del g
        spot_g = [from_torch(params[i].grad) for i in spot]
        big_g = [from_torch(params[i].grad) for i in big] if step < big_steps else None
        opt.step()
        torch.cuda.synchronize()
        orc.step(spot_g)
        bad += _compare_spot(opt, params, orc, spot, f"step {step + 1}")
        if big_g is not None:
            orc_big.step(big_g)
            bad += _compare_spot(opt, params, orc_big, big, f"step {step + 1}")
            del big_g
        log(f"  step {step + 1}: GPU step done, oracle spot checks {'ok' if not bad else 'FAILED'}")
        if bad:
            break
    bad += _invariants(opt, params, 4)
    assert not bad, "\n".join(bad[:20])


def test_gpt2_block_200_steps():
    """Config C0 as specified: one GPT-2-small block in fp32 (12 tensors,
    7,087,872 params; LayerNorm weights 1, the rest N(0, 0.02)), gradients
    N(0, s_t^2) with s_t ~ LogNormal(ln 1e-3, 1) per tensor plus a persistent
    drift direction of 0.3 s_t, v_bits 4, lr 6e-4, wd 0.01: 200 steps on the
    GPU, every tensor against the oracle bit for bit every 20 steps."""
    from turboadam_amd import TurboAdam

    shapes = bench.gpt2_block_shapes()
    log(f"C0: {len(shapes)} tensors, 200 steps")
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(17)
    params = []
    for name, shp in shapes:
        t = torch.ones(shp, device=dev) if name.startswith("ln_") and name.endswith(".w") else \
            torch.empty(shp, device=dev).normal_(0.0, 0.02, generator=gen)
        params.append(torch.nn.Parameter(t))
    kw = dict(lr=6e-4, weight_decay=0.01, v_bits=4)
    opt = TurboAdam(params, philox_seed=SEED, **kw)
    oparams = [from_torch(p) for p in params]
    orc = O.OracleTurboAdam(oparams, seed=SEED, **kw)
    sig = np.exp(math.log(1e-3) + np.random.default_rng(3).standard_normal(len(shapes)))
    drift = [torch.randn(shp, device=dev, generator=gen) for _, shp in shapes]
    for step in range(200):
        for i, p in enumerate(params):
            z = torch.randn(p.shape, device=dev, generator=gen)
            p.grad = (z + 0.3 * drift[i]) * float(sig[i])
        grads = [from_torch(p.grad) for p in params]
        opt.step()
        orc.step(grads)
        if (step + 1) % 20 == 0:
            torch.cuda.synchronize()
            bad = compare_with_oracle(opt, params, orc, oparams, f"step {step + 1}")
            log(f"  step {step + 1}: {'ok' if not bad else 'FAILED'}")
            assert not bad, "\n".join(bad[:20])
    assert all(int(opt.state[p]["step"]) == 200 for p in params)


def test_v_only_2_28_full_steps_sliced():
    """Config C1: one fp32 parameter of 2^28 elements, fp32 m, 4-bit v, its 50
    steps; three block-aligned slices (start, middle, end) against the oracle
    every 10 steps (only the slices travel to the host)."""
    from turboadam_amd import TurboAdam

    n = 1 << 28
    nb = n // 128
    slices = [(0, 64), (nb // 2 + 7, nb // 2 + 71), (nb - 64, nb)]
    steps = 50
    log(f"C1 full size: {n} elements, {steps} steps, slices {slices}")
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(9)
    p = torch.nn.Parameter(torch.empty(n, dtype=torch.float32, device=dev).normal_(0.0, 0.02, generator=gen))
    kw = dict(lr=1e-3, compress_m=False, v_bits=4)
    opt = TurboAdam([p], philox_seed=SEED, **kw)
    orc = O.OracleTurboAdam([from_torch(p.data[a * 128:b * 128]) for a, b in slices], seed=SEED,
                            tensor_ids=[0] * len(slices), block0=[a for a, _ in slices], **kw)
    bad = []
    for step in range(steps):
        p.grad = torch.randn(n, device=dev, generator=gen, dtype=torch.float32).mul_(1e-3)
        g = [from_torch(p.grad[a * 128:b * 128]) for a, b in slices]
        opt.step()
        orc.step(g)
        if (step + 1) % 10 and step != 0:
            continue
        torch.cuda.synchronize()
        st = opt.state[p]
        for j, (a, b) in enumerate(slices):
            ost = orc.state[j]
            where = f"step {step + 1} blocks [{a}, {b})"
            if not np.array_equal(_param_bits(p.data[a * 128:b * 128]),
                                  orc.param_groups[0]["params"][j].view(np.uint32)):
                bad.append(f"{where}: params differ")
            if not np.array_equal(from_torch(st["compressed_v"]["indices"][a * 128:b * 128]), ost["indices"]):
                bad.append(f"{where}: indices differ")
            if not np.array_equal(f16_bits(st["compressed_v"]["scales"].reshape(-1)[2 * a:2 * b]), ost["scales"]):
                bad.append(f"{where}: scales differ")
            if not np.array_equal(from_torch(st["exp_avg"][a * 128:b * 128]).view(np.uint32),
                                  ost["exp_avg"].view(np.uint32)):
                bad.append(f"{where}: exp_avg differs")
        log(f"  step {step + 1}: {'ok' if not bad else 'FAILED'}")
        if bad:
            break
    bad += _invariants(opt, [p], 4)
    assert not bad, "\n".join(bad[:20])


def test_gpt2_124m_sparse_embedding_full_steps():
    """Config C2: GPT-2 124M fp32 (148 tensors), Student-t(3) gradients, the
    token embedding with all but 5% of its rows exactly zero each step; the
    embedding, an MLP projection and a LayerNorm bias against the oracle at
    each of 20 steps."""
    from turboadam_amd import TurboAdam

    shapes = bench.gpt2_124m_shapes()
    names = [s[0] for s in shapes]
    spot = [names.index(k) for k in ("wte", "h11.mlp.c_proj.w", "ln_f.b")]
    steps = 20
    log(f"C2 full size: {len(shapes)} tensors, {steps} steps, spot checks {[names[i] for i in spot]}")
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(13)
    params = []
    for name, shp in shapes:
        if name.startswith("ln") or ".ln_" in name:
            t = torch.ones(shp, device=dev) if name.endswith(".w") else torch.zeros(shp, device=dev)
        else:
            t = torch.randn(shp, device=dev, generator=gen) * 0.02
        params.append(torch.nn.Parameter(t))
    kw = dict(lr=6e-4, weight_decay=0.1, v_bits=4)
    opt = TurboAdam(params, philox_seed=SEED, **kw)
    orc = O.OracleTurboAdam([from_torch(params[i]) for i in spot], seed=SEED, tensor_ids=spot, **kw)
    sig = np.exp(math.log(1e-3) + np.random.default_rng(2).standard_normal(len(shapes)))
    wte_rows = shapes[0][1][0]
    bad = []
    for step in range(steps):
        for i, (p, (name, shp)) in enumerate(zip(params, shapes)):
            # Student-t(3): z / sqrt(chi2_3 / 3), chi2_3 as a sum of three squared normals
            z = torch.randn(shp, device=dev, generator=gen)
            chi = sum(torch.randn(shp, device=dev, generator=gen) ** 2 for _ in range(3))
            g = z / torch.sqrt(chi / 3.0) * float(sig[i])
            if name == "wte":
                keep = torch.zeros(wte_rows, dtype=torch.bool, device=dev)
                keep[torch.randperm(wte_rows, generator=gen, device=dev)[: wte_rows // 20]] = True
                g[~keep] = 0.0
            p.grad = g
        spot_g = [from_torch(params[i].grad) for i in spot]
        opt.step()
        torch.cuda.synchronize()
        orc.step(spot_g)
        bad += _compare_spot(opt, params, orc, spot, f"step {step + 1}")
        log(f"  step {step + 1}: {'ok' if not bad else 'FAILED'}")
        if bad:
            break
    bad += _invariants(opt, params, 4)
    assert not bad, "\n".join(bad[:20])


@pytest.mark.parametrize("bits", [2, 3, 6, 8])
@pytest.mark.parametrize("pct", [(0.10, 0.90), (0.05, 0.95)])
def test_ragged_1000_tensors_full_steps(bits, pct):
    """Config C4: 1000 fp32 tensors of sizes round(2^(20U)) (CoState from 4096
    elements, tail blocks almost everywhere), each v_bits x percentile run;
    twelve tensors of every size class against the oracle."""
    from turboadam_amd import TurboAdam

    shapes = bench.ragged_shapes()
    sizes = np.array([s[1][0] for s in shapes])
    order = np.argsort(sizes, kind="stable")
    picks = [order[0], order[-1]]
    picks.append(int(np.flatnonzero(sizes < 128)[0]))
    picks.append(int(np.flatnonzero((sizes > 128) & (sizes < 4096) & (sizes % 128 != 0))[0]))
    picks.append(int(np.flatnonzero((sizes >= 4096) & (sizes % 128 != 0))[0]))
    picks.append(int(np.flatnonzero(sizes % 128 == 0)[0]))
    rng = np.random.default_rng(bits * 10 + int(pct[0] * 100))
    picks += [int(i) for i in rng.choice(len(shapes), 6, replace=False)]
    spot = sorted(set(int(i) for i in picks))
    log(f"C4 full size: {len(shapes)} tensors ({int(sizes.sum())} params), v_bits={bits}, pct={pct}, "
        f"spot sizes {[int(sizes[i]) for i in spot]}")
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(bits)
    params = [torch.nn.Parameter(torch.empty(s[1], device=dev).normal_(0.0, 0.02, generator=gen)) for s in shapes]
    kw = dict(lr=1e-3, v_bits=bits, null_pct=pct[0], amp_pct=pct[1])
    opt = TurboAdam(params, philox_seed=SEED + bits, **kw)
    orc = O.OracleTurboAdam([from_torch(params[i]) for i in spot], seed=SEED + bits, tensor_ids=spot, **kw)
    bad = []
    for step in range(4):
        for p in params:
            p.grad = torch.randn(p.shape, device=dev, generator=gen).mul_(1e-3)
        spot_g = [from_torch(params[i].grad) for i in spot]
        opt.step()
        torch.cuda.synchronize()
        orc.step(spot_g)
        bad += _compare_spot(opt, params, orc, spot, f"step {step + 1}")
    log(f"  4 steps: {'ok' if not bad else 'FAILED'}")
    bad += _invariants(opt, params, bits, *pct)
    assert not bad, "\n".join(bad[:20])


def test_ragged_1000_tensors_100_steps():
    """Config C4 for its 100 steps at one combination (v_bits 3, percentiles
    0.10 / 0.90): the twelve tensors of every size class against the oracle
    every 10 steps."""
    from turboadam_amd import TurboAdam

    bits, pct, steps = 3, (0.10, 0.90), 100
    shapes = bench.ragged_shapes()
    sizes = np.array([s[1][0] for s in shapes])
    order = np.argsort(sizes, kind="stable")
    picks = [order[0], order[-1], int(np.flatnonzero(sizes < 128)[0]),
             int(np.flatnonzero((sizes > 128) & (sizes < 4096) & (sizes % 128 != 0))[0]),
             int(np.flatnonzero((sizes >= 4096) & (sizes % 128 != 0))[0]), int(np.flatnonzero(sizes % 128 == 0)[0])]
    picks += [int(i) for i in np.random.default_rng(71).choice(len(shapes), 6, replace=False)]
    spot = sorted(set(int(i) for i in picks))
    log(f"C4 full size: {len(shapes)} tensors, {steps} steps, v_bits={bits}, pct={pct}, "
        f"spot sizes {[int(sizes[i]) for i in spot]}")
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(101)
    params = [torch.nn.Parameter(torch.empty(s[1], device=dev).normal_(0.0, 0.02, generator=gen)) for s in shapes]
    kw = dict(lr=1e-3, v_bits=bits, null_pct=pct[0], amp_pct=pct[1])
    opt = TurboAdam(params, philox_seed=SEED + 100, **kw)
    orc = O.OracleTurboAdam([from_torch(params[i]) for i in spot], seed=SEED + 100, tensor_ids=spot, **kw)
    bad = []
    for step in range(steps):
        for p in params:
            p.grad = torch.randn(p.shape, device=dev, generator=gen).mul_(1e-3)
        spot_g = [from_torch(params[i].grad) for i in spot]
        opt.step()
        orc.step(spot_g)
        if (step + 1) % 10 == 0:
            torch.cuda.synchronize()
            bad += _compare_spot(opt, params, orc, spot, f"step {step + 1}")
            log(f"  step {step + 1}: {'ok' if not bad else 'FAILED'}")
            if bad:
                break
    bad += _invariants(opt, params, bits, *pct)
    assert not bad, "\n".join(bad[:20])
