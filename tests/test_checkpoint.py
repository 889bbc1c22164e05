"""Checkpoints: the reference's format loads safely and is adopted (CPU).

The GPU tests (test_gpu_checkpoint.py) resume steps from such checkpoints;
these check the loading itself, which needs no device.
"""

import io
import pickle

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import reference_manager_class, reference_state_dict


def _oracle_after_steps(sizes, steps=2, seed=5):
    rng = np.random.default_rng(seed)
    params = [(rng.standard_normal(n) * 0.02).astype(np.float32) for n in sizes]
    orc = O.OracleTurboAdam(params, seed=seed, lr=1e-3, weight_decay=0.01)
    for _ in range(steps):
        orc.step([(rng.standard_normal(n) * 1e-3).astype(np.float32) for n in sizes])
    return orc


def _reference_checkpoint(orc, shapes) -> io.BytesIO:
    buf = io.BytesIO()
    with reference_manager_class() as ref_cls:
        torch.save(reference_state_dict(orc, shapes, ref_cls), buf)
    buf.seek(0)
    return buf


def test_reference_checkpoint_loads_with_weights_only_and_adopts():
    from turboadam_amd import TurboAdam, load_reference_checkpoint
    from turboadam_amd.costate import CoStateManager

    sizes, shapes = [5000, 300], [(50, 100), (300,)]
    orc = _oracle_after_steps(sizes)
    sd = load_reference_checkpoint(_reference_checkpoint(orc, shapes))
    assert isinstance(sd["state"][0]["m_mgr"], CoStateManager)
    assert "rand_buf" in sd["state"][0]["compressed_v"]
    params = [torch.nn.Parameter(torch.zeros(s)) for s in shapes]
    opt = TurboAdam(params, lr=1e-3, weight_decay=0.01)
    opt.load_state_dict(sd)
    st = opt.state[params[0]]
    mgr = st["m_mgr"]
    assert type(mgr) is CoStateManager and mgr._has_state and mgr._original_numel == 5000
    assert (mgr._null_pct, mgr._amp_pct, mgr.block_size) == (0.10, 0.90, 128)
    enc, ost = mgr._encoded, orc.state[0]
    assert enc["labels"].dtype == torch.uint8 and np.array_equal(enc["labels"].numpy(), ost["labels"])
    assert np.array_equal(enc["sign_packed"].numpy(), ost["sign_packed"])
    assert np.array_equal(enc["block_norms"].numpy().view(np.uint32), ost["block_norms"].view(np.uint32))
    assert enc["scales"].dtype == torch.float16
    assert np.array_equal(enc["scales"].view(torch.int16).numpy().view(np.uint16), ost["amp"])
    assert mgr._alpha.dtype == torch.float32 and float(mgr._alpha) == float(ost["alpha"][0])
    cv = st["compressed_v"]
    assert "rand_buf" not in cv and cv["indices"].dtype == torch.uint8 and cv["scales"].dtype == torch.float16
    assert np.array_equal(cv["scales"].reshape(-1).view(torch.int16).numpy().view(np.uint16), ost["scales"])
    small = opt.state[params[1]]
    assert "m_mgr" not in small and small["exp_avg"].dtype == torch.float32
    assert st["step"] == 2 and small["step"] == 2


class _NotAllowed:
    pass


def test_reference_loader_executes_nothing_from_the_file():
    from turboadam_amd import load_reference_checkpoint

    buf = io.BytesIO()
    torch.save({"state": {0: {"x": _NotAllowed()}}}, buf)
    buf.seek(0)
    with pytest.raises(pickle.UnpicklingError):
        load_reference_checkpoint(buf)


def test_state_dict_carries_the_philox_seed():
    from turboadam_amd import TurboAdam

    ps = [torch.nn.Parameter(torch.zeros(8))]
    sd = TurboAdam(ps, philox_seed=12345).state_dict()
    assert sd["philox_seed"] == 12345
    opt = TurboAdam(ps)
    opt.load_state_dict(sd)
    assert opt.philox_seed == 12345


def test_load_state_dict_keeps_fp32_moments_of_16bit_parameters():
    """torch's loader casts state tensors to the parameter dtype; the fp32
    exp_avg / exp_avg_sq of a bf16 parameter must come back unrounded."""
    from turboadam_amd import TurboAdam

    ps = [torch.nn.Parameter(torch.zeros(300, dtype=torch.bfloat16)),
          torch.nn.Parameter(torch.zeros(20, 10, dtype=torch.float16))]
    fine = torch.full((300,), 1.0 + 2.0 ** -20, dtype=torch.float32)
    sd = {"state": {0: {"step": 3, "_compress_m": False, "exp_avg": fine.clone(), "exp_avg_sq": fine * 2.0},
                    1: {"step": 3, "_compress_m": False, "exp_avg": fine[:200].reshape(20, 10) * 3.0,
                        "exp_avg_sq": fine[:200].reshape(20, 10) * 4.0}},
          "param_groups": [{**TurboAdam(ps).param_groups[0], "params": [0, 1], "compress_v": False}]}
    opt = TurboAdam([{"params": ps, "compress_v": False}])
    opt.load_state_dict(sd)
    for p, scale in zip(ps, (1.0, 3.0)):
        st = opt.state[p]
        for key, k in (("exp_avg", scale), ("exp_avg_sq", 2.0 if scale == 1.0 else 4.0)):
            t = st[key]
            assert t.dtype == torch.float32 and t.shape == p.shape
            want = (fine[: p.numel()] * k).reshape(p.shape)
            assert torch.equal(t, want), key
        assert st["step"] == 3
