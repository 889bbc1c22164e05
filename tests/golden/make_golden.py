"""Write golden fixtures from the reference implementation (run in the build container only).

    python tests/golden/make_golden.py /path/to/reference

Imports the reference package (davidkny22/turboadam, src/turboadam) from the
given checkout and runs its CPU path, TurboAdam.step(), on small synthetic
parameter sets.  Nothing of the reference is stored: the fixtures hold only
outputs (parameters and packed optimizer state, as arrays and per-step
SHA-1 digests) for inputs that oracle/inputs.py regenerates bit for bit.

The reference draws its stochastic-rounding uniforms with one call,
torch.rand_like(frac) in quantize.fused_v_update (quantize.py:291), once per
parameter with a gradient and in parameter order.  During the run that call
is replaced by the Philox4x32-10 stream of oracle/tam_oracle.c for
(tensor_id, step), so the reference consumes exactly the draws the GPU and the
oracle consume.  torch runs with one intra-op thread (its dot product depends
on the thread count).
"""

import hashlib
import json
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import inputs as I  # noqa: E402
from oracle import oracle as O  # noqa: E402

SR_SEED = 0x5EED_0000_2026_0001
TORCH_DT = {O.DT_F32: torch.float32, O.DT_BF16: torch.bfloat16, O.DT_F16: torch.float16}

GPT2_BLOCK = [(768,), (768,), (768, 2304), (2304,), (768, 768), (768,), (768,), (768,), (768, 3072), (3072,),
              (3072, 768), (768,)]

CASES = {
    "mv_f32": dict(sizes=[4096, 5000, 5123, 300, 1, 18432], dt=O.DT_F32, steps=8,
                   kw=dict(lr=6e-4, weight_decay=0.01)),
    "vonly_f32": dict(sizes=[9000, 300, 1, 4173], dt=O.DT_F32, steps=8, kw=dict(lr=1e-3, compress_m=False)),
    "mv_bf16": dict(sizes=[12288, 8320, 777], dt=O.DT_BF16, steps=6, kw=dict(lr=1e-3, weight_decay=0.1)),
    "mv_f16": dict(sizes=[8192, 1000], dt=O.DT_F16, steps=5, kw=dict(lr=1e-3)),
    "bits2": dict(sizes=[5096, 513], dt=O.DT_F32, steps=4, kw=dict(v_bits=2, null_pct=0.05, amp_pct=0.95)),
    "bits3": dict(sizes=[5096, 513], dt=O.DT_F32, steps=4, kw=dict(v_bits=3)),
    "bits6": dict(sizes=[5096, 513], dt=O.DT_F32, steps=4, kw=dict(v_bits=6, null_pct=0.05, amp_pct=0.95)),
    "bits8": dict(sizes=[5096, 513], dt=O.DT_F32, steps=4, kw=dict(v_bits=8)),
    "no_v": dict(sizes=[6000, 200], dt=O.DT_F32, steps=4, kw=dict(compress_v=False)),
    "adam": dict(sizes=[6000, 200], dt=O.DT_F32, steps=4, kw=dict(compress_m=False, compress_v=False)),
    "traj_f32": dict(sizes=[4608, 300], dt=O.DT_F32, steps=200, kw=dict(lr=1e-3, weight_decay=0.01),
                     keep_params=[25, 50, 100, 150, 200]),
    "gpt2_block": dict(sizes=[int(np.prod(s)) for s in GPT2_BLOCK], shapes=GPT2_BLOCK, dt=O.DT_F32, steps=3,
                       kw=dict(lr=6e-4, weight_decay=0.01), digests_only=True),
    # CoState error feedback (costate.py:409-437): the residual EMA is part of the state
    "ef_f32": dict(sizes=[5000, 4608, 300, 18509], dt=O.DT_F32, steps=8,
                   kw=dict(lr=1e-3, weight_decay=0.01, error_feedback=True)),
    "ef_bf16": dict(sizes=[8320, 4100], dt=O.DT_BF16, steps=6,
                    kw=dict(lr=1e-3, weight_decay=0.1, error_feedback=True, null_pct=0.05, amp_pct=0.95)),
}


def to_bits(x32: np.ndarray, dt: int) -> np.ndarray:
    if dt == O.DT_F32:
        return x32.astype(np.float32)
    return torch.from_numpy(x32.astype(np.float32)).to(TORCH_DT[dt]).view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray, dt: int) -> torch.Tensor:
    if dt == O.DT_F32:
        return torch.from_numpy(a.copy())
    return torch.from_numpy(a.view(np.int16).copy()).view(TORCH_DT[dt])


def np_of(t: torch.Tensor) -> np.ndarray:
    t = t.detach().reshape(-1).cpu()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def case_inputs(case):
    sizes = case["sizes"]
    init = [to_bits(a, case["dt"]) for a in I.param_init(sizes)]
    sig = I.grad_sigmas(len(sizes))
    return init, sig


def step_grads(case, sig, step):
    return [to_bits(g, case["dt"]) for g in I.grads(case["sizes"], step, sig)]


class PhiloxRandLike:
    """Stands in for torch.rand_like during a reference step."""

    def __init__(self, seed):
        self.seed = seed
        self.queue = []

    def __call__(self, t, *args, **kwargs):
        tid, step = self.queue.pop(0)
        u = O.philox_uniforms(tid, step, self.seed, t.numel())
        return torch.from_numpy(u).reshape(t.shape).to(dtype=t.dtype)


def state_arrays(opt, p) -> dict:
    st = opt.state[p]
    out = {}
    if "compressed_v" in st:
        out["indices"] = np_of(st["compressed_v"]["indices"].to(torch.uint8))
        out["scales"] = np_of(st["compressed_v"]["scales"].to(torch.float16))
    if st.get("_compress_m"):
        mgr = st["m_mgr"]
        enc = mgr._encoded
        out["labels"] = np_of(enc["labels"])
        out["sign_packed"] = np_of(enc["sign_packed"])
        out["block_norms"] = np_of(enc["block_norms"])
        out["amp"] = np_of(enc["scales"])
        out["alpha"] = np_of(mgr._alpha.reshape(1).float())
        if getattr(mgr, "_ef_residual", None) is not None:
            out["ef_residual"] = np_of(mgr._ef_residual.float())
    if "exp_avg" in st:
        out["exp_avg"] = np_of(st["exp_avg"])
    if "exp_avg_sq" in st:
        out["exp_avg_sq"] = np_of(st["exp_avg_sq"])
    return out


def digest(arrs: dict) -> str:
    h = hashlib.sha1()
    for k in sorted(arrs):
        h.update(k.encode())
        h.update(np.ascontiguousarray(arrs[k]).tobytes())
    return h.hexdigest()


def run_reference(ref_mod, name, case):
    torch.manual_seed(0)
    init, sig = case_inputs(case)
    shapes = case.get("shapes") or [(n,) for n in case["sizes"]]
    params = [torch.nn.Parameter(from_bits(a, case["dt"]).reshape(s)) for a, s in zip(init, shapes)]
    opt = ref_mod.TurboAdam(params, **case["kw"])
    rl = PhiloxRandLike(SR_SEED)
    orig = torch.rand_like
    out = {}
    digests = []
    compress_v = case["kw"].get("compress_v", True)
    try:
        torch.rand_like = rl
        for s in range(case["steps"]):
            grads = step_grads(case, sig, s)
            for p, g, shp in zip(params, grads, shapes):
                p.grad = from_bits(g, case["dt"]).reshape(shp)
            if compress_v:
                rl.queue = [(i, (opt.state[p]["step"] if p in opt.state and len(opt.state[p]) else 0) + 1)
                            for i, p in enumerate(params)]
            opt.step()
            if rl.queue:
                raise RuntimeError("reference did not draw the expected uniforms")
            step_d = []
            for i, p in enumerate(params):
                arrs = state_arrays(opt, p)
                arrs["param"] = np_of(p.data)
                step_d.append(digest(arrs))
                if s + 1 in case.get("keep_params", []):
                    out[f"p{s + 1}_{i}"] = arrs["param"]
            digests.append(step_d)
    finally:
        torch.rand_like = orig
    if not case.get("digests_only"):
        for i, p in enumerate(params):
            for k, v in state_arrays(opt, p).items():
                out[f"{k}_{i}"] = v
            out[f"param_{i}"] = np_of(p.data)
    else:
        # a sample of every tensor's final parameters (every 997th element)
        for i, p in enumerate(params):
            out[f"psample_{i}"] = np_of(p.data)[::997]
    meta = {"name": name, "sizes": case["sizes"], "dt": case["dt"], "steps": case["steps"], "kw": case["kw"],
            "shapes": [list(s) for s in shapes], "sr_seed": SR_SEED, "digests": digests,
            "keep_params": case.get("keep_params", []), "digests_only": bool(case.get("digests_only")),
            "torch": torch.__version__, "threads": torch.get_num_threads()}
    return out, meta


# Function-level fixtures of the 1Q quantizer (quantize.py:126-180 and
# oneq.py:13-48), which the step reaches only through its closed-form first
# state.  Inputs are stored with the outputs.
Q_CASES = {
    "q_det_b4": dict(n=128 * 64, bits=4, stochastic=False, fn="quantize"),
    "q_det_b2": dict(n=128 * 64, bits=2, stochastic=False, fn="quantize"),
    "q_sto_b3": dict(n=128 * 64, bits=3, stochastic=True, fn="quantize", tid=3, step=4),
    "q_sto_b8": dict(n=128 * 64, bits=8, stochastic=True, fn="quantize", tid=7, step=2),
    "compress_b4": dict(n=5000, bits=4, stochastic=False, fn="compress"),
}


def q_case_input(name, case):
    """Positive values spread over ~35 e-folds, some exact zeros (clamped to 1e-38)."""
    z = I.normal(case["n"], 77 + sorted(Q_CASES).index(name), 0)
    v = np.exp(-20.0 + 5.0 * z).astype(np.float32)
    v[::97] = 0.0
    return v


def run_reference_quantize(ref_mod, name, case):
    import importlib

    quant = importlib.import_module(ref_mod.__name__ + ".quantize")
    oneq = importlib.import_module(ref_mod.__name__ + ".oneq")
    v = q_case_input(name, case)
    rl = PhiloxRandLike(SR_SEED)
    orig = torch.rand_like
    try:
        torch.rand_like = rl
        if case["fn"] == "quantize":
            if case["stochastic"]:
                rl.queue = [(case["tid"], case["step"])]
            idx, scales, _ = quant.quantize_logscale_nbits(torch.from_numpy(v), n_bits=case["bits"], block_size=128,
                                                           stochastic_round=case["stochastic"])
        else:
            st = oneq.compress_v_logscale(torch.from_numpy(v), n_bits=case["bits"], block_size=128,
                                          stochastic_round=False)
            idx, scales = st["indices"], st["scales"]
    finally:
        torch.rand_like = orig
    out = {"v": v, "indices": np_of(idx.to(torch.uint8)), "scales": np_of(scales.to(torch.float16))}
    meta = {"name": name, **case, "sr_seed": SR_SEED, "torch": torch.__version__, "threads": torch.get_num_threads()}
    return out, meta


# The 1Q decode (quantize.py:183-214, oneq.py:51-67) of the reference's own
# quantizer outputs above: all values, and a trimmed count.
DEQ_TRIM = 37


def run_reference_dequantize(ref_mod):
    import importlib

    quant = importlib.import_module(ref_mod.__name__ + ".quantize")
    oneq = importlib.import_module(ref_mod.__name__ + ".oneq")
    out, cases = {}, {}
    for name, case in Q_CASES.items():
        z = np.load(os.path.join(HERE, f"golden_{name}.npz"))
        idx = torch.from_numpy(z["indices"].copy())
        scales = torch.from_numpy(z["scales"].view(np.int16).copy()).view(torch.float16).reshape(-1, 2)
        nb = scales.shape[0]
        full = quant.dequantize_logscale_nbits(idx, scales, n_bits=case["bits"], block_size=128, original_numel=0)
        trim = quant.dequantize_logscale_nbits(idx, scales, n_bits=case["bits"], block_size=128,
                                               original_numel=nb * 128 - DEQ_TRIM)
        out[f"{name}_full"] = np_of(full)
        out[f"{name}_trim"] = np_of(trim)
        if case["fn"] == "compress":
            st = {"indices": idx, "scales": scales, "n_bits": case["bits"], "original_shape": torch.Size([case["n"]]),
                  "original_length": case["n"], "block_size": 128}
            out[f"{name}_decompress"] = np_of(oneq.decompress_v(st))
        cases[name] = {"bits": case["bits"], "nb": nb}
    meta = {"cases": cases, "trim": DEQ_TRIM, "torch": torch.__version__, "threads": torch.get_num_threads()}
    return out, meta


# Host logic the other cases leave out (optimizer.py:224-292, :172-188, and
# torch.optim's add_param_group): two groups with their own hyperparameters,
# gradients that are None for some steps (a parameter first stepped late,
# which as its group's last parameter with state sets the group's shared bias
# corrections; a stepped parameter then skipped), and a third group added
# before step 5.
GROUPS_CASE = dict(
    sizes=[5000, 300, 4608, 9000, 2000], dt=O.DT_F32, steps=8,
    groups=[dict(idx=[0, 1], kw=dict(lr=1e-3, weight_decay=0.01)),
            dict(idx=[2, 3], kw=dict(lr=5e-4, betas=(0.8, 0.99), v_bits=3, null_pct=0.05, amp_pct=0.95))],
    added=dict(before_step=4, idx=[4], kw=dict(lr=2e-3, weight_decay=0.1, compress_m=False)),
    kw=dict(lr=1e-3),
    # step (0-based) -> parameters without a gradient
    none={0: [3], 1: [1, 3], 2: [1, 3]},
)


def groups_grads(case, sig, s):
    """Gradients of step s (None where the schedule gives none, or before a
    parameter's group exists)."""
    gs = step_grads(case, sig, s)
    added = case["added"]
    return [None if (i in case["none"].get(s, []) or (i in added["idx"] and s < added["before_step"])) else g
            for i, g in enumerate(gs)]


def run_reference_groups(ref_mod, case=GROUPS_CASE):
    torch.manual_seed(0)
    init, sig = case_inputs(case)
    params = [torch.nn.Parameter(from_bits(a, case["dt"])) for a in init]
    opt = ref_mod.TurboAdam([{"params": [params[i] for i in g["idx"]], **g["kw"]} for g in case["groups"]],
                            **case["kw"])
    order = [i for g in case["groups"] for i in g["idx"]]
    rl = PhiloxRandLike(SR_SEED)
    orig = torch.rand_like
    digests = []
    try:
        torch.rand_like = rl
        for s in range(case["steps"]):
            if s == case["added"]["before_step"]:
                opt.add_param_group({"params": [params[i] for i in case["added"]["idx"]], **case["added"]["kw"]})
                order += case["added"]["idx"]
            grads = groups_grads(case, sig, s)
            for i, p in enumerate(params):
                p.grad = None if grads[i] is None else from_bits(grads[i], case["dt"])
            # tensor ids are positions in param_groups order (here equal to the indices)
            # (opt.state is a defaultdict: a parameter without state must not be looked up,
            # or the reference's next _prepare_step_scalars finds an empty state)
            rl.queue = [(order.index(i), (opt.state[params[i]]["step"] if params[i] in opt.state else 0) + 1)
                        for i in order if grads[i] is not None]
            opt.step()
            if rl.queue:
                raise RuntimeError("reference did not draw the expected uniforms")
            step_d = []
            for i, p in enumerate(params):
                arrs = state_arrays(opt, p) if p in opt.state else {}
                arrs["param"] = np_of(p.data)
                step_d.append(digest(arrs))
            digests.append(step_d)
    finally:
        torch.rand_like = orig
    out = {}
    for i, p in enumerate(params):
        for k, v in state_arrays(opt, p).items():
            out[f"{k}_{i}"] = v
        out[f"param_{i}"] = np_of(p.data)
        out[f"step_{i}"] = np.array(opt.state[p]["step"])
    meta = {"name": "groups", "digests": digests, "sr_seed": SR_SEED, "torch": torch.__version__,
            "threads": torch.get_num_threads()}
    return out, meta


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    only = sys.argv[2:]  # optional case names
    sys.path.insert(0, os.path.join(ref_root, "src"))
    import turboadam as ref_mod  # the reference package

    torch.set_num_threads(1)
    for name, case in CASES.items():
        if only and name not in only:
            continue
        out, meta = run_reference(ref_mod, name, case)
        path = os.path.join(HERE, f"golden_{name}.npz")
        np.savez_compressed(path, meta=np.array(json.dumps(meta)), **out)
        print(f"{name}: {os.path.getsize(path)} bytes", flush=True)
    for name, case in Q_CASES.items():
        if only and name not in only:
            continue
        out, meta = run_reference_quantize(ref_mod, name, case)
        path = os.path.join(HERE, f"golden_{name}.npz")
        np.savez_compressed(path, meta=np.array(json.dumps(meta)), **out)
        print(f"{name}: {os.path.getsize(path)} bytes", flush=True)
    for name, fn in (("dequantize", run_reference_dequantize), ("groups", run_reference_groups)):
        if only and name not in only:
            continue
        out, meta = fn(ref_mod)
        path = os.path.join(HERE, f"golden_{name}.npz")
        np.savez_compressed(path, meta=np.array(json.dumps(meta)), **out)
        print(f"{name}: {os.path.getsize(path)} bytes", flush=True)


if __name__ == "__main__":
    main()
