"""GradScaler (torch.amp) interplay on the GPU, bit for bit.

TurboAdam declares _step_supports_amp_scaling: GradScaler hands it grad_scale
and found_inf instead of unscaling and reading found_inf on the host.  The
results must equal GradScaler's default flow for other optimizers (unscale_
then a host-side skip), including the skipped steps and the scale schedule.
For capturable groups the skip happens on the device: a captured step replays
as a skip whenever found_inf is nonzero, counters included.  Gradients are
fp32: GradScaler's unscale op has no bf16 kernel on this torch build (it
raises for bf16 gradients before the optimizer is reached, with or without
this protocol).  The oracle steps on the unscaled gradients of the steps
that are not skipped (scales are powers of two, so unscaling is exact) and
must equal both flows bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import compare_states, compare_with_oracle, from_torch, gpu_state, log, to_bits, to_torch

pytestmark = pytest.mark.gpu

F32 = O.DT_F32


def _bits(a):
    return a.view(np.uint32) if a.dtype == np.float32 else a


def _compare(opt_a, pa, opt_b, pb, where, steps_a=None):
    bad = []
    for i, (a, b) in enumerate(zip(pa, pb)):
        if not np.array_equal(_bits(from_torch(a)), _bits(from_torch(b))):
            bad.append(f"{where} tensor {i}: params differ")
        if b in opt_b.state:
            bad += compare_states(gpu_state(opt_a, a), gpu_state(opt_b, b), f"{where} tensor {i}")
            sa, sb = opt_a.state[a]["step"], opt_b.state[b]["step"]
            if int(sa) != int(sb):
                bad.append(f"{where} tensor {i}: step {int(sa)} vs {int(sb)}")
        elif a in opt_a.state and int(opt_a.state[a]["step"]) != 0:
            bad.append(f"{where} tensor {i}: stepped although the reference never did")
    return bad


def _setup(seed):
    sizes = [70_001, 5000, 300]
    dts = [F32, F32, F32]
    rng = np.random.default_rng(seed)
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
    grads = [[(rng.standard_normal(n) * 1e-3).astype(np.float32) for n in sizes] for _ in range(7)]
    return sizes, dts, init, grads


def test_grad_scaler_protocol_equals_default_flow():
    from turboadam_amd import TurboAdam

    dev = torch.device("cuda:0")
    sizes, dts, init, grads = _setup(41)
    pa = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    pb = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    kw = dict(lr=1e-3, weight_decay=0.05, philox_seed=5)
    opt_a = TurboAdam(pa, **kw)
    opt_b = TurboAdam(pb, **kw)
    opt_b._step_supports_amp_scaling = False  # GradScaler: unscale_, host check, skip
    oparams = [a.copy() for a in init]
    orc = O.OracleTurboAdam(oparams, dtypes=dts, seed=5, lr=1e-3, weight_decay=0.05)
    sc_a = torch.amp.GradScaler("cuda", init_scale=2.0 ** 12, growth_interval=2)
    sc_b = torch.amp.GradScaler("cuda", init_scale=2.0 ** 12, growth_interval=2)
    one = torch.ones((), device=dev)
    sc_a.scale(one)
    sc_b.scale(one)
    for s, gs in enumerate(grads):
        scale = float(sc_a.get_scale())
        assert scale == float(sc_b.get_scale())
        for params in (pa, pb):
            for i, (p, g, dt, n) in enumerate(zip(params, gs, dts, sizes)):
                gg = (g * np.float32(scale)).astype(np.float32)
                if s in (1, 4) and i == 0:
                    gg[7] = np.inf  # an overflowed step: skipped, the scale halves
                p.grad = to_torch(to_bits(gg, dt), dt, (n,), dev)
        sc_a.step(opt_a)
        sc_a.update()
        sc_b.step(opt_b)
        sc_b.update()
        if s not in (1, 4):
            orc.step([to_bits(g, dt) for g, dt in zip(gs, dts)])
        torch.cuda.synchronize()
        log(f"amp step {s + 1}: scale {scale}")
        bad = _compare(opt_a, pa, opt_b, pb, f"step {s + 1}")
        bad += compare_with_oracle(opt_a, pa, orc, oparams, f"step {s + 1} vs oracle", sizes)
        assert not bad, "\n".join(bad[:20])


def test_captured_step_skips_on_device_when_found_inf():
    from turboadam_amd import TurboAdam

    dev = torch.device("cuda:0")
    sizes, dts, init, grads = _setup(42)
    pc = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    pe = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    kw = dict(lr=1e-3, weight_decay=0.05, philox_seed=6)
    cap = TurboAdam(pc, capturable=True, **kw)
    eager = TurboAdam(pe, **kw)
    eager._step_supports_amp_scaling = False
    oparams = [a.copy() for a in init]
    orc = O.OracleTurboAdam(oparams, dtypes=dts, seed=6, lr=1e-3, weight_decay=0.05)
    scale = torch.full((), 2.0 ** 8, dtype=torch.float32, device=dev)
    found = torch.zeros((), dtype=torch.float32, device=dev)
    static = [torch.zeros(n, dtype=p.dtype, device=dev) for n, p in zip(sizes, pc)]
    skips = [False, True, False, False, True, True, False]

    def set_static(s):
        for st, g, dt, n in zip(static, grads[s], dts, sizes):
            st.copy_(to_torch(to_bits((g * np.float32(256.0)).astype(np.float32), dt), dt, (n,), dev))
        found.fill_(1.0 if skips[s] else 0.0)
        for p, st in zip(pc, static):
            p.grad = st

    def eager_step(s):
        for p, g, dt, n in zip(pe, grads[s], dts, sizes):
            p.grad = to_torch(to_bits((g * np.float32(256.0)).astype(np.float32), dt), dt, (n,), dev)
        inv = scale.double().reciprocal().float()
        torch._amp_foreach_non_finite_check_and_unscale_([p.grad for p in pe], torch.zeros(1, device=dev), inv)
        if not skips[s]:
            eager.step()
            orc.step([to_bits(g, dt) for g, dt in zip(grads[s], dts)])

    cap.grad_scale, cap.found_inf = scale, found
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for s in range(2):  # warm-up: a step, then a skipped one
            set_static(s)
            cap.step()
    torch.cuda.current_stream().wait_stream(side)
    for s in range(2):
        eager_step(s)
    torch.cuda.synchronize()
    bad = _compare(cap, pc, eager, pe, "warm-up") + compare_with_oracle(cap, pc, orc, oparams, "warm-up vs oracle")
    assert not bad, "\n".join(bad[:20])
    graph = torch.cuda.CUDAGraph()
    set_static(2)
    with torch.cuda.graph(graph):
        cap.step()
    torch.cuda.synchronize()
    for s in range(2, len(grads)):
        set_static(s)
        graph.replay()
        eager_step(s)
        torch.cuda.synchronize()
        torch.randn(1 << 20, device=dev).sum().item()  # eager work between replays
        log(f"replay {s - 1}: skip={skips[s]}")
        bad = _compare(cap, pc, eager, pe, f"replay {s - 1}")
        bad += compare_with_oracle(cap, pc, orc, oparams, f"replay {s - 1} vs oracle", sizes)
        assert not bad, "\n".join(bad[:20])
    del cap.grad_scale, cap.found_inf
