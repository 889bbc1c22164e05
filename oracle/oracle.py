"""TEST INFRASTRUCTURE ONLY -- the CPU oracle of the TurboAdam step.

Never imported by the turboadam_amd package.  tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg use it as the checker.

`OracleTurboAdam` restates the host logic of the reference optimizer
(davidkny22/turboadam src/turboadam/optimizer.py:88-292: lazy state init,
bias corrections shared per group with the last parameter's value, step
counters, small-tensor routing to an fp32 exp_avg) over numpy arrays and calls
the exact-mode C restatement (oracle/tam_oracle.c) for each parameter.
Parameters of dtype bf16 / f16 are held as uint16 bit patterns.
"""

import ctypes
import math
import os

import numpy as np

from .build import LIB_PATH, build_oracle

DT_F32, DT_BF16, DT_F16 = 0, 1, 2
FLAG_COSTATE, FLAG_COMPRESS_V, FLAG_HAS_STATE, FLAG_WD, FLAG_EF, FLAG_HAS_EF = 1, 2, 4, 8, 16, 32
BS = 128
# f16(log(f32(1e-30))): the initial 1Q scale (reference oneq.py:13-48 on full(1e-30)).
V_INIT_SCALE_BITS = np.float16(-69.0625).view(np.uint16)

_VP = ctypes.c_void_p


class OrTensor(ctypes.Structure):
    _fields_ = [
        ("param", _VP), ("grad", _VP), ("v_idx", _VP), ("v_scales", _VP), ("exp_avg_sq", _VP),
        ("exp_avg", _VP), ("signs", _VP), ("labels", _VP), ("norms", _VP), ("amp", _VP), ("alpha", _VP),
        ("ef_residual", _VP), ("n", ctypes.c_uint64),
        ("dtype", ctypes.c_uint32), ("flags", ctypes.c_uint32), ("v_bits", ctypes.c_uint32),
        ("tensor_id", ctypes.c_uint32), ("step", ctypes.c_uint32), ("k_lo", ctypes.c_uint32),
        ("k_hi", ctypes.c_uint32), ("block0", ctypes.c_uint32),
        ("c_wd", ctypes.c_float), ("beta1", ctypes.c_float), ("one_minus_beta1", ctypes.c_float),
        ("beta2", ctypes.c_float), ("one_minus_beta2", ctypes.c_float), ("bias_correction1", ctypes.c_float),
        ("bias_correction2", ctypes.c_float), ("eps", ctypes.c_float), ("neg_lr", ctypes.c_float),
        ("sqrt_block", ctypes.c_float),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build_oracle()
        L = ctypes.CDLL(LIB_PATH)
        L.or_step_tensor.argtypes = [ctypes.POINTER(OrTensor), ctypes.c_uint64]
        L.or_philox_uniforms.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint64, _VP]
        L.or_input_uniforms.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint64, _VP]
        L.or_philox4x32_10.argtypes = [_VP, ctypes.c_uint32, ctypes.c_uint32, _VP]
        L.or_logf.argtypes = [ctypes.c_float]
        L.or_logf.restype = ctypes.c_float
        L.or_expf.argtypes = [ctypes.c_float]
        L.or_expf.restype = ctypes.c_float
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_bf16.argtypes = [ctypes.c_float]
        L.or_f32_to_bf16.restype = ctypes.c_uint16
        L.or_pairwise_sum.argtypes = [_VP, ctypes.c_uint64]
        L.or_pairwise_sum.restype = ctypes.c_double
        L.or_thresholds.argtypes = [_VP, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64, _VP, _VP]
        L.or_decompose.argtypes = [_VP, _VP, ctypes.c_uint64, _VP]
        L.or_decompose.restype = ctypes.c_float
        L.or_block_ratios.argtypes = [_VP, _VP, ctypes.c_uint64, _VP]
        L.or_classify.argtypes = [_VP, ctypes.c_uint64, ctypes.c_float, ctypes.c_float, _VP]
        L.or_encode.argtypes = [_VP, ctypes.c_uint64, ctypes.c_float, _VP, _VP, _VP]
        L.or_decode_blocks.argtypes = [_VP, _VP, _VP, _VP, ctypes.c_float, _VP, ctypes.c_uint64, ctypes.c_float, _VP]
        L.or_fused_v_update.argtypes = [_VP, _VP, _VP, ctypes.c_uint64, ctypes.c_int, ctypes.c_float,
                                        ctypes.c_float, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64, _VP]
        L.or_dequantize.argtypes = [_VP, _VP, ctypes.c_uint64, ctypes.c_int, _VP]
        L.or_quantize_logscale.argtypes = [_VP, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_uint32,
                                           ctypes.c_uint32, ctypes.c_uint64, _VP, _VP]
        L.or_costate_update.argtypes = [_VP, ctypes.c_uint64, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                        ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, _VP, _VP, _VP, _VP, _VP, _VP]
        L.or_costate_update_ef.argtypes = [_VP, ctypes.c_uint64, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                           ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, _VP, _VP, _VP, _VP, _VP,
                                           ctypes.c_int, ctypes.c_int, _VP, _VP]
        L.or_struct_size.restype = ctypes.c_size_t
        if L.or_struct_size() != ctypes.sizeof(OrTensor):
            raise RuntimeError("oracle struct layout mismatch")
        _lib = L
    return _lib


def ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def f32(x: float) -> float:
    return float(np.float32(x))


def philox_uniforms(tensor_id: int, step: int, seed: int, count: int) -> np.ndarray:
    """The stochastic-rounding uniforms of (tensor_id, step) for elements 0 .. count-1."""
    out = np.empty(count, dtype=np.float32)
    lib().or_philox_uniforms(tensor_id, step, seed, count, ptr(out))
    return out


def input_uniforms(stream: int, draw: int, seed: int, count: int) -> np.ndarray:
    """Uniforms of the synthetic test inputs (another bit layout of the same generator)."""
    out = np.empty(count, dtype=np.float32)
    lib().or_input_uniforms(stream, draw, seed, count, ptr(out))
    return out


def dequantize(indices: np.ndarray, scales_bits: np.ndarray, n: int, bits: int) -> np.ndarray:
    """or_dequantize: the first n decoded 1Q values (scales as f16 bit patterns, 2 per block)."""
    idx = np.ascontiguousarray(indices, dtype=np.uint8)
    sc = np.ascontiguousarray(scales_bits, dtype=np.uint16).reshape(-1)
    if n > idx.size or (n + BS - 1) // BS > sc.size // 2:
        raise ValueError("dequantize: state does not cover n values")
    out = np.empty(n, np.float32)
    lib().or_dequantize(ptr(idx), ptr(sc), n, bits, ptr(out))
    return out


def ranks(nb: int, null_pct: float, amp_pct: float):
    return max(0, int(null_pct * nb) - 1), min(nb - 1, int(amp_pct * nb))


DEFAULTS = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, block_size=128, v_bits=4,
                compress_m=True, compress_v=True, null_pct=0.10, amp_pct=0.90, error_feedback=False,
                min_m_compress_elements=4096)


class OracleTurboAdam:
    """Host logic of reference TurboAdam.step over numpy parameters.

    params: list of numpy arrays (float32, or uint16 bit patterns with the
    matching entry of `dtypes` = DT_BF16 / DT_F16), or a list of groups
    {"params": [...], **hyperparameters}.  tensor_ids: the Philox tensor id of
    each parameter (default: its position, as TurboAdam numbers them);
    block0: for a parameter that is a block-aligned slice of a larger one
    without CoState, the slice's first block (its draws are then that
    parameter's).
    """

    def __init__(self, params, dtypes=None, seed=0, tensor_ids=None, block0=None, **kw):
        if params and isinstance(params[0], dict):
            groups = params
        else:
            groups = [{"params": list(params)}]
        self.defaults = dict(DEFAULTS)
        self.defaults.update(kw)
        self.param_groups = []
        flat = []
        for g in groups:
            grp = dict(self.defaults)
            grp.update({k: v for k, v in g.items() if k != "params"})
            grp["params"] = list(g["params"])
            flat.extend(grp["params"])
            self.param_groups.append(grp)
        self.dtypes = list(dtypes) if dtypes is not None else [DT_F32] * len(flat)
        self.tensor_ids = list(tensor_ids) if tensor_ids is not None else list(range(len(flat)))
        self.block0 = list(block0) if block0 is not None else [0] * len(flat)
        self.seed = seed
        self.state = {}

    def add_param_group(self, group, dtypes=None):
        """torch.optim.Optimizer.add_param_group: a new group whose unset
        hyperparameters are the optimizer's defaults; its parameters follow all
        earlier ones (their Philox tensor ids continue the numbering)."""
        grp = dict(self.defaults)
        grp.update({k: v for k, v in group.items() if k != "params"})
        grp["params"] = list(group["params"])
        n0 = len(self.dtypes)
        self.param_groups.append(grp)
        self.dtypes += list(dtypes) if dtypes is not None else [DT_F32] * len(grp["params"])
        self.tensor_ids += list(range(n0, n0 + len(grp["params"])))
        self.block0 += [0] * len(grp["params"])

    def _init(self, pid, p, grp):
        n = p.size
        nb = (n + BS - 1) // BS
        st = {"step": 0}
        st["_compress_m"] = bool(grp["compress_m"] and n >= grp["min_m_compress_elements"])
        if st["_compress_m"]:
            st["labels"] = np.zeros(nb, np.uint8)
            st["sign_packed"] = np.zeros((n + 7) // 8, np.uint8)
            st["block_norms"] = np.zeros(nb, np.float32)
            st["amp"] = np.zeros(nb, np.uint16)
            st["alpha"] = np.zeros(1, np.float32)
            st["has_state"] = False
            if grp["error_feedback"]:  # costate.py:409-437: the residual appears after the first update
                st["ef_residual"] = np.zeros(n, np.float32)
                st["has_ef"] = False
        else:
            st["exp_avg"] = np.zeros(n, np.float32)
        if not grp["compress_v"]:
            st["exp_avg_sq"] = np.zeros(n, np.float32)
        else:
            st["indices"] = np.zeros(nb * BS, np.uint8)
            st["scales"] = np.full(nb * 2, V_INIT_SCALE_BITS, np.uint16)
        self.state[pid] = st

    def step(self, grads):
        """grads: list aligned with the flattened parameter list (None = no gradient)."""
        L = lib()
        pid = 0
        entries = []
        for gi, grp in enumerate(self.param_groups):
            for p in grp["params"]:
                g = grads[pid]
                if g is not None:
                    if pid not in self.state:
                        self._init(pid, p, grp)
                    entries.append((pid, gi, grp, p, g))
                pid += 1
        # bias corrections: last parameter with state in the group (optimizer.py:172-188)
        bc = {}
        pid = 0
        for gi, grp in enumerate(self.param_groups):
            b1, b2 = grp["betas"]
            for p in grp["params"]:
                if pid in self.state:
                    nxt = self.state[pid]["step"] + 1
                    bc[gi] = (1.0 - b1**nxt, 1.0 - b2**nxt)
                pid += 1
        for pid, gi, grp, p, g in entries:
            st = self.state[pid]
            st["step"] += 1
            n = p.size
            nb = (n + BS - 1) // BS
            t = OrTensor()
            t.param = ptr(p)
            t.grad = ptr(g)
            t.n = n
            t.dtype = self.dtypes[pid]
            flags = 0
            if grp["compress_v"]:
                flags |= FLAG_COMPRESS_V
                t.v_idx = ptr(st["indices"])
                t.v_scales = ptr(st["scales"])
                t.v_bits = grp["v_bits"]
            else:
                t.exp_avg_sq = ptr(st["exp_avg_sq"])
            if st["_compress_m"]:
                flags |= FLAG_COSTATE
                if st["has_state"]:
                    flags |= FLAG_HAS_STATE
                t.signs = ptr(st["sign_packed"])
                t.labels = ptr(st["labels"])
                t.norms = ptr(st["block_norms"])
                t.amp = ptr(st["amp"])
                t.alpha = ptr(st["alpha"])
                if "ef_residual" in st:
                    flags |= FLAG_EF | (FLAG_HAS_EF if st["has_ef"] else 0)
                    t.ef_residual = ptr(st["ef_residual"])
                t.k_lo, t.k_hi = ranks(nb, grp["null_pct"], grp["amp_pct"])
            else:
                t.exp_avg = ptr(st["exp_avg"])
            lr, wd = grp["lr"], grp["weight_decay"]
            b1, b2 = grp["betas"]
            if wd != 0.0:
                flags |= FLAG_WD
            t.flags = flags
            t.tensor_id = self.tensor_ids[pid]
            t.block0 = self.block0[pid]
            t.step = st["step"]
            c1, c2 = bc[gi]
            t.c_wd = f32(1.0 - lr * wd)
            t.beta1, t.one_minus_beta1 = f32(b1), f32(1.0 - b1)
            t.beta2, t.one_minus_beta2 = f32(b2), f32(1.0 - b2)
            t.bias_correction1, t.bias_correction2 = f32(c1), f32(c2)
            t.eps = f32(grp["eps"])
            t.neg_lr = f32(-lr)
            t.sqrt_block = f32(math.sqrt(BS))
            L.or_step_tensor(ctypes.byref(t), self.seed)
            if st["_compress_m"]:
                st["has_state"] = True
                if "ef_residual" in st:
                    st["has_ef"] = True
