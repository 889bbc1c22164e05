"""The optimizer class's API behaviours on the GPU, each checked bit for bit
against the CPU oracle (reference behaviours: tests/test_optimizer.py:492-513
closure, :585-611 fp16 and autocast, :620-663 gradient accumulation,
:669-713 add_param_group, :722-740 min_m_compress_elements routing).

Gradients come from real autograd passes through small torch modules on the
GPU; the oracle steps on copies of exactly the gradients the optimizer saw.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import compare_with_oracle, from_torch, log

pytestmark = pytest.mark.gpu

DT = {torch.float32: O.DT_F32, torch.bfloat16: O.DT_BF16, torch.float16: O.DT_F16}


def _oracle_for(params, seed=0, **kw):
    """The oracle on copies of params' current values (same dtypes and Philox key)."""
    oparams = [from_torch(p.data) for p in params]
    orc = O.OracleTurboAdam(oparams, dtypes=[DT[p.dtype] for p in params], seed=seed, **kw)
    return orc, oparams


def _grads(params):
    return [None if p.grad is None else from_torch(p.grad) for p in params]


def _model(dtype=torch.float32, width=128):
    torch.manual_seed(0)
    m = torch.nn.Sequential(torch.nn.Linear(width, 64), torch.nn.GELU(), torch.nn.Linear(64, 8))
    return m.to(device="cuda:0", dtype=dtype)


def test_step_with_closure_returns_its_loss():
    """step(closure) evaluates the closure with gradients enabled, returns its
    loss, and steps on the gradients the closure produced."""
    from turboadam_amd import TurboAdam

    model = _model()
    params = list(model.parameters())  # 8192-element weight: CoState; the rest fp32 m
    opt = TurboAdam(params, lr=1e-2, weight_decay=0.01, philox_seed=11)
    orc, oparams = _oracle_for(params, seed=11, lr=1e-2, weight_decay=0.01)
    x = torch.randn(32, 128, device="cuda:0")
    seen = {}
    for s in range(4):
        def closure():
            opt.zero_grad()
            loss = model(x).square().mean()
            loss.backward()
            seen["loss"] = loss
            seen["grads"] = _grads(params)
            return loss

        with torch.no_grad():  # the closure must still get gradients
            loss = opt.step(closure)
        assert loss is seen["loss"]
        assert float(loss.detach()) > 0
        orc.step(seen["grads"])
        torch.cuda.synchronize()
        bad = compare_with_oracle(opt, params, orc, oparams, f"closure step {s + 1}")
        assert not bad, "\n".join(bad[:20])
    assert opt.step() is None  # no closure, no loss


def test_gradient_accumulation_steps_once():
    """Gradients accumulated over several backward passes give one step: the
    step counter moves by one and the update is the oracle's single step on
    the summed gradient; weight decay applies once per step."""
    from turboadam_amd import TurboAdam

    model = _model()
    params = list(model.parameters())
    opt = TurboAdam(params, lr=1e-2, weight_decay=0.1, philox_seed=12)
    orc, oparams = _oracle_for(params, seed=12, lr=1e-2, weight_decay=0.1)
    xs = [torch.randn(16, 128, device="cuda:0") for _ in range(3)]
    for s in range(3):
        opt.zero_grad(set_to_none=False)
        for x in xs:
            model(x * (s + 1)).square().mean().backward()
        for p in params:
            assert int(opt.state[p]["step"]) == s if p in opt.state else s == 0
        orc.step(_grads(params))
        opt.step()
        torch.cuda.synchronize()
        for p in params:
            assert int(opt.state[p]["step"]) == s + 1
        bad = compare_with_oracle(opt, params, orc, oparams, f"accumulated step {s + 1}")
        assert not bad, "\n".join(bad[:20])

    # zero gradients over three accumulations: only the decay moves the
    # parameters, once: p * (1 - lr * wd), rounded once per element
    ones = torch.nn.Parameter(torch.ones(10, 10, device="cuda:0"))
    opt1 = TurboAdam([ones], lr=1e-2, weight_decay=0.1)
    for _ in range(3):
        opt1.zero_grad()
        ones.grad = torch.zeros_like(ones)
    opt1.step()
    want = np.float32(1.0) * (np.float32(1.0) - np.float32(1e-2) * np.float32(0.1))
    assert np.array_equal(from_torch(ones.data), np.full(100, want, np.float32))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_half_precision_parameters(dtype):
    """16-bit parameters with 16-bit gradients from autograd (CoState and fp32-m
    tensors alike) step as the oracle does."""
    from turboadam_amd import TurboAdam

    model = _model(dtype)
    params = list(model.parameters())
    opt = TurboAdam(params, lr=1e-3, weight_decay=0.01, philox_seed=13)
    orc, oparams = _oracle_for(params, seed=13, lr=1e-3, weight_decay=0.01)
    x = torch.randn(32, 128, device="cuda:0", dtype=dtype)
    for s in range(4):
        opt.zero_grad()
        model(x).float().square().mean().backward()
        assert all(p.grad.dtype == dtype for p in params)
        orc.step(_grads(params))
        opt.step()
        torch.cuda.synchronize()
        bad = compare_with_oracle(opt, params, orc, oparams, f"{dtype} step {s + 1}")
        assert not bad, "\n".join(bad[:20])
        assert all(bool(torch.isfinite(p).all()) for p in params)


def test_autocast_forward():
    """fp32 parameters with a forward pass under torch.autocast (fp16 matmuls):
    the fp32 gradients autograd produces step as the oracle does."""
    from turboadam_amd import TurboAdam

    model = _model()
    params = list(model.parameters())
    opt = TurboAdam(params, lr=1e-3, philox_seed=14)
    orc, oparams = _oracle_for(params, seed=14, lr=1e-3)
    x = torch.randn(32, 128, device="cuda:0")
    for s in range(3):
        opt.zero_grad()
        with torch.autocast("cuda", dtype=torch.float16):
            loss = model(x).square().mean()
        loss.float().backward()
        assert all(p.grad.dtype == torch.float32 for p in params)
        orc.step(_grads(params))
        opt.step()
        torch.cuda.synchronize()
        bad = compare_with_oracle(opt, params, orc, oparams, f"autocast step {s + 1}")
        assert not bad, "\n".join(bad[:20])


@pytest.mark.parametrize("threshold", [100, 200, 5000, 5001])
def test_min_m_compress_elements_routing(threshold):
    """A tensor takes CoState when its size reaches min_m_compress_elements,
    an fp32 exp_avg below it (reference optimizer.py:245-248)."""
    from turboadam_amd import TurboAdam

    rng = np.random.default_rng(threshold)
    sizes = [100, 200, 5000]
    params = [torch.nn.Parameter(torch.from_numpy((rng.standard_normal(n) * 0.02).astype(np.float32)).cuda())
              for n in sizes]
    opt = TurboAdam(params, lr=1e-3, min_m_compress_elements=threshold, philox_seed=15)
    orc, oparams = _oracle_for(params, seed=15, lr=1e-3, min_m_compress_elements=threshold)
    for s in range(3):
        for p in params:
            p.grad = torch.from_numpy((rng.standard_normal(p.numel()) * 1e-3).astype(np.float32)).cuda()
        orc.step(_grads(params))
        opt.step()
        torch.cuda.synchronize()
        bad = compare_with_oracle(opt, params, orc, oparams, f"threshold {threshold} step {s + 1}")
        assert not bad, "\n".join(bad[:20])
    for p, n in zip(params, sizes):
        st = opt.state[p]
        if n >= threshold:
            assert "m_mgr" in st and "exp_avg" not in st and st["_compress_m"]
        else:
            assert "exp_avg" in st and "m_mgr" not in st and not st["_compress_m"]


def test_add_param_group_mid_run():
    """A group added after five steps starts its own step count at one, with
    its own lr; the first group's bias corrections continue (6 steps)."""
    from turboadam_amd import TurboAdam

    rng = np.random.default_rng(16)
    x = torch.nn.Parameter(torch.from_numpy((rng.standard_normal(6000) * 0.02).astype(np.float32)).cuda())
    y = torch.nn.Parameter(torch.from_numpy((rng.standard_normal(5000) * 0.02).astype(np.float32)).cuda())
    opt = TurboAdam([x], lr=1e-2, philox_seed=17)
    oparams = [from_torch(x.data), from_torch(y.data)]
    orc = O.OracleTurboAdam([oparams[0]], seed=17, lr=1e-2)
    for s in range(5):
        opt.zero_grad()
        (x.square().sum() * (1 + s)).backward()
        orc.step(_grads([x]))
        opt.step()
    opt.add_param_group({"params": [y], "lr": 1e-3})
    orc.add_param_group({"params": [oparams[1]], "lr": 1e-3})
    opt.zero_grad()
    (x.square().sum() + y.square().sum()).backward()
    orc.step(_grads([x, y]))
    opt.step()
    torch.cuda.synchronize()
    assert int(opt.state[x]["step"]) == 6 and int(opt.state[y]["step"]) == 1
    log("add_param_group: steps 6 and 1")
    bad = compare_with_oracle(opt, [x, y], orc, oparams, "after add_param_group")
    assert not bad, "\n".join(bad[:20])
