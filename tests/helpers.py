"""Shared helpers: run the GPU TurboAdam and the CPU oracle side by side."""

import contextlib
import sys
import types

import numpy as np
import torch

from oracle import oracle as O

TORCH_DT = {O.DT_F32: torch.float32, O.DT_BF16: torch.bfloat16, O.DT_F16: torch.float16}


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def to_bits(x: np.ndarray, dt: int) -> np.ndarray:
    """fp32 numpy -> oracle representation of dtype dt (fp32 or uint16 bits, RNE)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dt == O.DT_F32:
        return x.copy()
    t = torch.from_numpy(x).to(TORCH_DT[dt])
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def to_torch(a: np.ndarray, dt: int, shape, device) -> torch.Tensor:
    if dt == O.DT_F32:
        t = torch.from_numpy(a.copy())
    else:
        t = torch.from_numpy(a.view(np.int16).copy()).view(TORCH_DT[dt])
    return t.reshape(shape).to(device)


def from_torch(t: torch.Tensor) -> np.ndarray:
    t = t.detach().reshape(-1).cpu()
    if t.dtype == torch.float32:
        return t.numpy().copy()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    if t.dtype == torch.uint8:
        return t.numpy().copy()
    raise TypeError(t.dtype)


def f16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().reshape(-1).cpu().view(torch.int16).numpy().view(np.uint16).copy()


def gpu_state(opt, p) -> dict:
    """Numpy view of a GPU TurboAdam parameter state in the oracle's key names."""
    st = opt.state[p]
    out = {"step": st["step"], "_compress_m": st["_compress_m"]}
    if st["_compress_m"]:
        mgr = st["m_mgr"]
        enc = mgr._encoded
        out["labels"] = from_torch(enc["labels"])
        out["sign_packed"] = from_torch(enc["sign_packed"])
        out["block_norms"] = from_torch(enc["block_norms"])
        out["amp"] = f16_bits(enc["scales"])
        out["alpha"] = from_torch(mgr._alpha.reshape(1))
        out["has_state"] = mgr._has_state
        if getattr(mgr, "_ef_residual", None) is not None:
            out["ef_residual"] = from_torch(mgr._ef_residual.float())
    else:
        out["exp_avg"] = from_torch(st["exp_avg"])
    if "exp_avg_sq" in st:
        out["exp_avg_sq"] = from_torch(st["exp_avg_sq"])
    if "compressed_v" in st:
        out["indices"] = from_torch(st["compressed_v"]["indices"])
        out["scales"] = f16_bits(st["compressed_v"]["scales"])
    return out


STATE_KEYS = ["labels", "sign_packed", "block_norms", "amp", "alpha", "exp_avg", "exp_avg_sq", "indices", "scales",
              "ef_residual"]


def compare_states(gst: dict, ost: dict, where: str) -> list:
    """Bit-exact comparison; returns a list of mismatch descriptions."""
    bad = []
    for k in STATE_KEYS:
        if k not in ost:
            continue
        a = gst.get(k)
        b = ost[k]
        if a is None:
            bad.append(f"{where}: {k} missing on GPU")
            continue
        if a.shape != b.shape:
            bad.append(f"{where}: {k} shape {a.shape} vs {b.shape}")
            continue
        av = a.view(np.uint32) if a.dtype == np.float32 else a
        bv = b.view(np.uint32) if b.dtype == np.float32 else b
        nd = int(np.count_nonzero(av != bv))
        if nd:
            i = int(np.flatnonzero(av != bv)[0])
            bad.append(f"{where}: {k} differs in {nd}/{a.size} (first at {i}: gpu {a[i]} oracle {b[i]})")
    return bad


def make_grads(rng, sizes, dts, sigmas, drifts=None, drift_scale=0.3):
    out = []
    for i, n in enumerate(sizes):
        g = rng.standard_normal(n).astype(np.float32) * np.float32(sigmas[i])
        if drifts is not None:
            g = g + np.float32(drift_scale * sigmas[i]) * drifts[i]
        out.append(to_bits(g.astype(np.float32), dts[i]))
    return out


def _at_offset(t: torch.Tensor, offset: int) -> torch.Tensor:
    """A copy of t that starts `offset` elements into a larger allocation."""
    if not offset:
        return t
    base = torch.zeros(t.numel() + offset, dtype=t.dtype, device=t.device)
    view = base[offset:].view(t.shape)
    view.copy_(t)
    return view


def run_side_by_side(sizes, dts, steps, seed=0, check_every=1, shapes=None, grad_none=None, offset=0, **kw):
    """Step the GPU optimizer and the oracle on identical inputs; return mismatch list.

    offset > 0 places every parameter and gradient that many elements into a
    larger allocation (unaligned arrays)."""
    from turboadam_amd import TurboAdam

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(seed)
    shapes = shapes or [(n,) for n in sizes]
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dts[i]) for i, n in enumerate(sizes)]
    o_params = [a.copy() for a in init]
    g_params = [torch.nn.Parameter(_at_offset(to_torch(a, dts[i], shapes[i], dev), offset))
                for i, a in enumerate(init)]
    opt = TurboAdam(g_params, **kw)
    opt.philox_seed = 1234567 + seed
    orc = O.OracleTurboAdam(o_params, dtypes=dts, seed=1234567 + seed, **kw)
    sigmas = np.exp(np.log(1e-3) + rng.standard_normal(len(sizes)))
    drifts = [rng.standard_normal(n).astype(np.float32) for n in sizes]
    bad = []
    for s in range(steps):
        grads = make_grads(rng, sizes, dts, sigmas, drifts)
        if grad_none is not None:
            grads = [None if grad_none(s, i) else g for i, g in enumerate(grads)]
        for i, p in enumerate(g_params):
            p.grad = None if grads[i] is None else _at_offset(to_torch(grads[i], dts[i], shapes[i], dev), offset)
        opt.step()
        orc.step(grads)
        if (s + 1) % check_every == 0 or s == steps - 1:
            torch.cuda.synchronize()
            bad += compare_with_oracle(opt, g_params, orc, o_params, f"step {s + 1}", sizes)
            if bad:
                return bad
    return bad


def _bits_of(a: np.ndarray) -> np.ndarray:
    return a.view(np.uint32) if a.dtype == np.float32 else a


def compare_with_oracle(opt, params, orc, o_params, where: str, sizes=None) -> list:
    """Parameters, every state array and the step counters of a GPU TurboAdam
    against the oracle's, bit for bit (the GPU's device-side step counters of
    a capturable group included); returns a list of mismatch descriptions."""
    bad = []
    for i, p in enumerate(params):
        w = f"{where} tensor {i}" + (f" (n={sizes[i]})" if sizes is not None else "")
        pa, pb = from_torch(p.data), o_params[i]
        if not np.array_equal(_bits_of(pa), _bits_of(pb)):
            nd = int(np.count_nonzero(_bits_of(pa) != _bits_of(pb)))
            bad.append(f"{w}: param differs in {nd}/{pa.size}")
        if i not in orc.state:
            if p in opt.state and int(opt.state[p]["step"]) != 0:
                bad.append(f"{w}: stepped on the GPU, never in the oracle")
            continue
        if p not in opt.state:
            bad.append(f"{w}: no GPU state")
            continue
        if int(opt.state[p]["step"]) != int(orc.state[i]["step"]):
            bad.append(f"{w}: step {int(opt.state[p]['step'])} vs oracle {orc.state[i]['step']}")
        bad += compare_states(gpu_state(opt, p), orc.state[i], w)
    return bad


REFERENCE_MANAGER_ATTRS = ("block_size", "_null_pct", "_amp_pct", "_has_state", "_alpha", "_encoded",
                           "_original_numel", "_error_feedback", "_ef_residual")


@contextlib.contextmanager
def reference_manager_class():
    """A class that pickles under the reference's name
    turboadam.costate.CoStateManager, for writing checkpoints in the reference's
    format (its state dict pickles the manager's attribute dict,
    costate.py:357-365) without the reference package."""
    pkg, mod = types.ModuleType("turboadam"), types.ModuleType("turboadam.costate")

    class CoStateManager:
        pass

    CoStateManager.__module__ = "turboadam.costate"
    CoStateManager.__qualname__ = "CoStateManager"
    mod.CoStateManager = CoStateManager
    pkg.costate = mod
    saved = {k: sys.modules.get(k) for k in ("turboadam", "turboadam.costate")}
    sys.modules["turboadam"], sys.modules["turboadam.costate"] = pkg, mod
    try:
        yield CoStateManager
    finally:
        for k, v in saved.items():
            if v is None:
                sys.modules.pop(k, None)
            else:
                sys.modules[k] = v


def reference_state_dict(orc, shapes, ref_cls, device="cpu"):
    """The reference optimizer's state_dict (optimizer.py:238-286 layout) for
    the oracle's current state: CoState managers as ref_cls objects, the 1Q
    dict with a rand_buf, shared bias-correction tensors."""
    state, pid = {}, 0
    bc = (torch.zeros(1), torch.zeros(1))
    groups = []
    for grp in orc.param_groups:
        ids = []
        for p in grp["params"]:
            if pid in orc.state:
                st = orc.state[pid]
                n = p.size
                nb = (n + O.BS - 1) // O.BS
                out = {"step": st["step"], "_compress_m": st["_compress_m"], "_bc1": bc[0], "_bc2": bc[1]}
                if st["_compress_m"]:
                    m = ref_cls()
                    m.block_size, m._null_pct, m._amp_pct = O.BS, grp["null_pct"], grp["amp_pct"]
                    m._has_state, m._original_numel = bool(st["has_state"]), n
                    m._error_feedback, m._ef_residual = False, None
                    m._alpha = torch.tensor(float(st["alpha"][0]), dtype=torch.float32)
                    m._encoded = {
                        "labels": torch.from_numpy(st["labels"].copy()),
                        "sign_packed": torch.from_numpy(st["sign_packed"].copy()),
                        "block_norms": torch.from_numpy(st["block_norms"].copy()),
                        "scales": torch.from_numpy(st["amp"].view(np.int16).copy()).view(torch.float16),
                    }
                    out["m_mgr"] = m
                else:
                    out["exp_avg"] = torch.from_numpy(st["exp_avg"].copy()).reshape(shapes[pid])
                if "exp_avg_sq" in st:
                    out["exp_avg_sq"] = torch.from_numpy(st["exp_avg_sq"].copy()).reshape(shapes[pid])
                if "indices" in st:
                    out["compressed_v"] = {
                        "indices": torch.from_numpy(st["indices"].copy()),
                        "scales": torch.from_numpy(st["scales"].view(np.int16).copy()).view(torch.float16)
                                       .reshape(nb, 2),
                        "n_bits": grp["v_bits"], "original_shape": torch.Size(shapes[pid]), "original_length": n,
                        "block_size": O.BS, "rand_buf": torch.zeros(nb * O.BS),
                    }
                state[pid] = out
            ids.append(pid)
            pid += 1
        g = {k: v for k, v in grp.items() if k != "params"}
        g["params"] = ids
        groups.append(g)
    return {"state": state, "param_groups": groups}
