"""A capturable step captured in a HIP graph and replayed (GPU).

With capturable=True the step's first launch takes the step number, the bias
corrections and the has-state flags from device counters, so one captured
step() replays as a real step each time.  Every replay, with new gradients
copied into the captured gradient tensors and eager work and synchronisations
between replays, must equal an eager optimizer's step and the CPU oracle's bit for
bit: parameters, every state array and the step counters (the device prologue's
step numbers, shared bias corrections and has-state flags are thereby checked
against the reference's host logic as the oracle restates it).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import compare_states, compare_with_oracle, from_torch, gpu_state, log, to_bits, to_torch

pytestmark = pytest.mark.gpu

F32, BF16 = O.DT_F32, O.DT_BF16


def _bits(a):
    return a.view(np.uint32) if a.dtype == np.float32 else a


def test_captured_step_replays_equal_eager_steps():
    from turboadam_amd import TurboAdam

    dev = torch.device("cuda:0")
    # group 0: CoState bf16 and fp32 (tails), an fp32-m tensor, and a tensor whose
    # first gradient comes at step 2 (the group's step counts then differ);
    # group 1: error feedback
    sizes = [70_001, 5000, 300, 9000, 12_345]
    dts = [BF16, F32, F32, BF16, F32]
    rng = np.random.default_rng(31)
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
    steps = 8
    grads = [[to_bits((rng.standard_normal(n) * 1e-3).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
             for _ in range(steps)]
    late = 3  # no gradient at step 1

    def groups(params):
        return [{"params": params[:4]}, {"params": params[4:], "error_feedback": True}]

    pe = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    pc = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    kw = dict(lr=1e-3, weight_decay=0.05, philox_seed=777)
    eager = TurboAdam(groups(pe), **kw)
    cap = TurboAdam(groups(pc), capturable=True, **kw)
    static = [torch.zeros_like(p) for p in pc]
    oparams = [a.copy() for a in init]
    orc = O.OracleTurboAdam(groups(oparams), dtypes=dts, seed=777, lr=1e-3, weight_decay=0.05)

    def step_oracle(s):
        orc.step([None if (i == late and s == 0) else g for i, g in enumerate(grads[s])])

    def set_eager(s):
        for i, (p, g, dt, n) in enumerate(zip(pe, grads[s], dts, sizes)):
            p.grad = None if (i == late and s == 0) else to_torch(g, dt, (n,), dev)

    def set_static(s):
        for i, (p, st, g, dt, n) in enumerate(zip(pc, static, grads[s], dts, sizes)):
            st.copy_(to_torch(g, dt, (n,), dev))
            p.grad = None if (i == late and s == 0) else st

    def compare(where):
        bad = []
        for i, (a, b) in enumerate(zip(pe, pc)):
            if not np.array_equal(_bits(from_torch(a)), _bits(from_torch(b))):
                bad.append(f"{where} tensor {i}: params differ")
            if a in eager.state:
                bad += compare_states(gpu_state(cap, b), gpu_state(eager, a), f"{where} tensor {i}")
                if int(cap.state[b]["step"].item()) != eager.state[a]["step"]:
                    bad.append(f"{where} tensor {i}: step counter differs")
        return bad + compare_with_oracle(cap, pc, orc, oparams, f"{where} vs oracle", sizes)

    # warm-up (eager) steps of the capturable optimizer on a side stream
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for s in range(2):
            set_static(s)
            cap.step()
    torch.cuda.current_stream().wait_stream(side)
    for s in range(2):
        set_eager(s)
        eager.step()
        step_oracle(s)
    torch.cuda.synchronize()
    bad = compare("warm-up")
    assert not bad, "\n".join(bad[:20])

    graph = torch.cuda.CUDAGraph()
    set_static(2)
    with torch.cuda.graph(graph):
        cap.step()
    torch.cuda.synchronize()
    log("captured one step; replaying")
    for s in range(2, steps):
        set_static(s)
        graph.replay()
        set_eager(s)
        eager.step()
        step_oracle(s)
        torch.cuda.synchronize()
        # eager work of the program's own between replays
        torch.randn(1 << 20, device=dev).sum().item()
        bad = compare(f"replay {s - 1}")
        assert not bad, "\n".join(bad[:20])


def test_steps_on_alternating_streams_equal_one_stream():
    """The descriptor and workspace buffers are reused from step to step; a step
    issued on another stream than the previous one is ordered after it."""
    from turboadam_amd import TurboAdam

    dev = torch.device("cuda:0")
    sizes = [4_000_003, 70_001, 5000, 300]
    dts = [BF16, BF16, F32, F32]
    rng = np.random.default_rng(33)
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
    steps = 6
    grads = [[to_torch(to_bits((rng.standard_normal(n) * 1e-3).astype(np.float32), dt), dt, (n,), dev)
              for n, dt in zip(sizes, dts)] for _ in range(steps)]
    pa = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    pb = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    kw = dict(lr=1e-3, weight_decay=0.05, philox_seed=99)
    oa, ob = TurboAdam(pa, **kw), TurboAdam(pb, **kw)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    main = torch.cuda.current_stream()
    for s in range(steps):
        for p, g in zip(pa, grads[s]):
            p.grad = g
        oa.step()
        st = streams[s % 2]
        st.wait_stream(main)  # the gradients were written on the main stream
        with torch.cuda.stream(st):
            for p, g in zip(pb, grads[s]):
                p.grad = g
            ob.step()
    for st in streams:
        main.wait_stream(st)
    torch.cuda.synchronize()
    log(f"{steps} steps, alternating streams")
    bad = []
    for i, (a, b) in enumerate(zip(pa, pb)):
        if not np.array_equal(_bits(from_torch(a)), _bits(from_torch(b))):
            bad.append(f"tensor {i}: params differ")
        bad += compare_states(gpu_state(ob, b), gpu_state(oa, a), f"tensor {i}")
    assert not bad, "\n".join(bad[:20])


def test_capturable_eager_steps_follow_a_betas_change():
    """Eager steps of a capturable optimizer whose betas change mid-run: the
    bias corrections come from the device table of the betas in force (the
    descriptor table is rebuilt for the new betas), as the oracle computes
    them from the group's betas at each step."""
    from turboadam_amd import TurboAdam

    dev = torch.device("cuda:0")
    sizes = [5000, 300, 9000]
    dts = [F32, F32, BF16]
    rng = np.random.default_rng(33)
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
    params = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    kw = dict(lr=1e-3, weight_decay=0.01)
    opt = TurboAdam(params, capturable=True, philox_seed=778, **kw)
    oparams = [a.copy() for a in init]
    orc = O.OracleTurboAdam(oparams, dtypes=list(dts), seed=778, **kw)
    for step in range(6):
        if step == 3:
            opt.param_groups[0]["betas"] = (0.8, 0.99)
            orc.param_groups[0]["betas"] = (0.8, 0.99)
        gs = [to_bits((rng.standard_normal(n) * 1e-3).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
        for p, g, dt, n in zip(params, gs, dts, sizes):
            p.grad = to_torch(g, dt, (n,), dev)
        opt.step()
        orc.step(gs)
        torch.cuda.synchronize()
        bad = compare_with_oracle(opt, params, orc, oparams, f"step {step + 1}", sizes)
        assert not bad, "\n".join(bad[:20])
    log("6 eager capturable steps, betas changed before step 4")
