"""CPU: the C-ABI library loads, exports every symbol include/turboadam_amd.h
declares, agrees with the Python struct mirror, and its host-only planning
(tam_prepare) validates input and lays out tiles and workspace.  No GPU call.
"""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from turboadam_amd import _lib
from turboadam_amd.build import LIB_PATH, REPO_DIR

HEADER = os.path.join(REPO_DIR, "include", "turboadam_amd.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tam_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB_PATH)
    names = _declared()
    assert len(names) >= 9
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), "binding and header disagree"


def test_load_checks_abi_and_struct_layout():
    lib = _lib.load()
    assert lib.tam_abi_version() == _lib.ABI_VERSION
    assert lib.tam_struct_size(0) == ctypes.sizeof(_lib.TamTensor) == 272
    assert lib.tam_struct_size(1) == ctypes.sizeof(_lib.TamStepInfo)


def _tensor(n, costate=True, compress_v=True, bits=4):
    t = _lib.TamTensor()
    t.param, t.grad = 0x10000, 0x20000
    t.n = n
    t.dtype = _lib.TAM_DTYPE_F32
    t.flags = (_lib.TAM_FLAG_COSTATE if costate else 0) | (_lib.TAM_FLAG_COMPRESS_V if compress_v else 0)
    t.v_idx, t.v_scales, t.v_bits = 0x30000, 0x40000, bits
    t.exp_avg_sq = t.exp_avg = 0x50000
    t.signs = t.labels = t.norms = t.amp = t.alpha = 0x60000
    nb = (n + 127) // 128
    t.k_lo, t.k_hi = max(0, int(0.1 * nb) - 1), min(nb - 1, int(0.9 * nb))
    t.sqrt_block = np.float32(np.sqrt(128.0))
    t.neg_lr, t.bias_correction1 = np.float32(-3e-4), np.float32(1.0 - 0.9 ** 3)
    return t


def _prepare(ts):
    lib = _lib.load()
    arr = (_lib.TamTensor * len(ts))(*ts)
    info = _lib.TamStepInfo()
    rc = lib.tam_prepare(arr, len(ts), ctypes.byref(info))
    return rc, arr, info, lib.tam_last_error().decode()


def test_prepare_layout():
    rc, arr, info, _ = _prepare([_tensor(5000), _tensor(300, costate=False), _tensor(2048 * 16 + 1)])
    assert rc == 0
    assert [a.nb for a in arr] == [40, 3, 257]
    assert [a.ntiles for a in arr] == [3, 1, 17]
    assert [a.tile0 for a in arr] == [0, 3, 4]
    assert info.total_tiles == 21 and info.n_costate == 2 and info.ratio_blocks == 40 + 260
    assert arr[0].ratio_off == 0 and arr[2].ratio_off == 40
    assert info.off_partials == 0
    assert info.off_alpha >= 21 * 4 * 16 and info.off_ratios >= info.off_alpha + 3 * 4
    assert info.ws_bytes >= info.off_ratios + 300 * 4
    # one alpha-reduction chunk per CoState tensor here (at most 8192 quarter-tile partials)
    assert info.total_chunks == 2 and [a.chunk0 for a in arr] == [0, 1, 1]
    assert info.off_chunks >= info.off_ratios + 300 * 4 and info.ws_bytes >= info.off_chunks + 2 * 16
    assert info.off_alpha % 256 == 0 and info.off_ratios % 256 == 0
    # derived: fl(-lr / bc1) as an fp32 division
    assert np.float32(arr[0].c_lr) == np.float32(-3e-4) / np.float32(1.0 - 0.9 ** 3)


@pytest.mark.parametrize("mutate,msg", [
    (lambda t: setattr(t, "n", 0), "no elements"),
    (lambda t: setattr(t, "v_bits", 5), "v_bits"),
    (lambda t: setattr(t, "dtype", 7), "dtype"),
    (lambda t: setattr(t, "alpha", 0), "CoState"),
    (lambda t: setattr(t, "v_idx", 0x30001), "misaligned"),
    (lambda t: setattr(t, "v_idx", 0x30008), "misaligned v state"),  # pass 0 loads 16 bytes per lane
    (lambda t: setattr(t, "v_scales", 0x40002), "misaligned v state"),
    (lambda t: setattr(t, "signs", 0x60001), "misaligned CoState"),
    (lambda t: setattr(t, "norms", 0x60002), "misaligned CoState"),
    (lambda t: setattr(t, "amp", 0x60001), "misaligned CoState"),
    (lambda t: setattr(t, "alpha", 0x60002), "misaligned CoState"),
    (lambda t: setattr(t, "k_hi", 10_000), "rank"),
    (lambda t: setattr(t, "sqrt_block", 11.0), "sqrt_block"),
    (lambda t: setattr(t, "found_inf", 0x4000), "found_inf"),  # a skip flag needs DEVICE_STEP
])
def test_prepare_rejects_bad_input(mutate, msg):
    t = _tensor(5000)
    mutate(t)
    rc, _, _, err = _prepare([t])
    assert rc == 1 and msg in err


def test_prepare_requires_one_found_inf_for_all_tensors():
    # the launches test descriptor 0's skip flag for the whole step
    ts = [_tensor(5000), _tensor(300)]
    for t in ts:
        t.flags |= _lib.TAM_FLAG_DEVICE_STEP
        t.step_dev = t.bc_step = t.bc_table = 0x4000
        t.bc_len = 1
    ts[0].found_inf = 0x5000
    rc, _, _, err = _prepare(ts)
    assert rc == 1 and "found_inf" in err
    ts[1].found_inf = 0x5000
    rc, arr, _, _ = _prepare(ts)
    assert rc == 0 and arr[0].flags & 0x80 == 0  # TAM_FLAG_SKIP is set on the device only


def test_optimizer_declares_amp_scaling_support():
    from turboadam_amd import TurboAdam

    assert TurboAdam._step_supports_amp_scaling is True


def test_step_rejects_small_workspace_without_launching():
    lib = _lib.load()
    rc, arr, info, _ = _prepare([_tensor(5000)])
    assert rc == 0
    rc = lib.tam_multi_tensor_step(0x1000, arr, ctypes.byref(info), 0, 0x2000, info.ws_bytes - 1, None)
    assert rc == 2 and "workspace" in lib.tam_last_error().decode()


def test_optimizer_refuses_cpu_parameters():
    from turboadam_amd import TurboAdam

    p = torch.nn.Parameter(torch.randn(10))
    opt = TurboAdam([p])
    p.grad = torch.randn(10)
    with pytest.raises(RuntimeError, match="HIP"):
        opt.step()


def test_constructor_validation_matches_reference():
    from turboadam_amd import TurboAdam

    ps = [torch.nn.Parameter(torch.randn(10, 10))]
    with pytest.raises(ValueError, match="v_bits must be one of"):
        TurboAdam(ps, v_bits=10)
    # the reference raises for capturable=True (optimizer.py:63-66); here the
    # step can be captured in a HIP graph (tests/test_gpu_capture.py)
    assert TurboAdam(ps, capturable=True).defaults["capturable"] is True
    opt = TurboAdam(ps)
    assert opt.defaults["capturable"] is False
    d = opt.defaults
    assert (d["lr"], d["betas"], d["eps"], d["weight_decay"], d["block_size"], d["v_bits"]) == \
        (1e-3, (0.9, 0.999), 1e-8, 0.0, 128, 4)
    assert d["compress_m"] is True and d["compress_v"] is True
    assert (d["null_pct"], d["amp_pct"], d["min_m_compress_elements"]) == (0.10, 0.90, 4096)


def test_philox_seed_keyword():
    from turboadam_amd import TurboAdam
    from turboadam_amd.quantize import DEFAULT_SEED

    ps = [torch.nn.Parameter(torch.randn(4))]
    assert TurboAdam(ps).philox_seed == DEFAULT_SEED
    assert TurboAdam(ps, philox_seed=(1 << 64) - 1).philox_seed == (1 << 64) - 1
    with pytest.raises(ValueError, match="philox_seed"):
        TurboAdam(ps, philox_seed=-1)
    with pytest.raises(TypeError):
        TurboAdam(ps, 1e-3, (0.9, 0.999), 1e-8, 0.0, 128, 4, True, True, 0.1, 0.9, False, False, 4096, 7)


def test_steady_step_sees_replaced_or_reset_state():
    """The steady path's state check (TurboAdam._fast_state_kept): a replaced
    state tensor, a reset per-parameter dict or a cleared opt.state make the
    next step take the full path; an unchanged state passes.  The state is
    built on the CPU in the optimizer's layout (no step runs here)."""
    from turboadam_amd.costate import CoStateManager
    from turboadam_amd.optimizer import TurboAdam, _FastStep, _row_tensors, _tensor_ptrs

    params = [torch.nn.Parameter(torch.zeros(n)) for n in (5000, 300)]
    opt = TurboAdam(params)
    for p in params:
        st = opt.state[p]
        st["step"] = 3
        st["compressed_v"] = {"indices": torch.zeros(128 * ((p.numel() + 127) // 128), dtype=torch.uint8),
                              "scales": torch.zeros(2 * ((p.numel() + 127) // 128), dtype=torch.float16)}
        st["_compress_m"] = p.numel() >= 4096
        if st["_compress_m"]:
            mgr = st["m_mgr"] = CoStateManager()
            mgr.allocate(p.numel(), torch.device("cpu"))
        else:
            st["exp_avg"] = torch.zeros(p.numel())

    class Plan:
        row_cv = [True, True]

    def fast():
        states = [opt.state[p] for p in params]
        return _FastStep(0, torch.device("cuda", 0), params, [True, True], [0, 1], states, [None, None],
                         [torch.float32] * 2, [], Plan, opt.state)

    assert opt._fast_state_kept(fast())
    replace = [
        lambda: opt.state[params[1]].__setitem__("exp_avg", torch.zeros(300)),
        lambda: opt.state[params[0]]["compressed_v"].__setitem__("indices", torch.zeros(5120, dtype=torch.uint8)),
        lambda: opt.state[params[1]]["compressed_v"].__setitem__("scales", torch.zeros(6, dtype=torch.float16)),
        lambda: opt.state[params[0]]["m_mgr"]._encoded.__setitem__("labels", torch.zeros(40, dtype=torch.uint8)),
        lambda: setattr(opt.state[params[0]]["m_mgr"], "_alpha", torch.zeros(())),
        lambda: opt.state.__setitem__(params[0], {}),
        lambda: opt.state.clear(),
    ]
    for k, change in enumerate(replace):
        f = fast()
        saved = {p: dict(opt.state[p]) for p in params}
        mgr = opt.state[params[0]]["m_mgr"]
        saved_mgr = (mgr._alpha, dict(mgr._encoded))
        change()
        assert not opt._fast_state_kept(f), k
        for p in params:  # restore for the next case
            opt.state[p] = saved[p]
        mgr._alpha, mgr._encoded = saved_mgr[0], saved_mgr[1]
        for p in params:
            opt.state[p]["compressed_v"] = dict(saved[p]["compressed_v"])
    # the full path compares device addresses of the same tensors
    rows = [_row_tensors(opt.state[p], True) for p in params]
    assert len(_tensor_ptrs(rows)) == 8 + 3 and _tensor_ptrs(rows)[7] == 0  # no error-feedback residual
