"""TurboAdam: Adam/AdamW with CoState-compressed m and 1Q-compressed v, stepped
by fused gfx950 kernels.

Drop-in for the reference class (davidkny22/turboadam,
src/turboadam/optimizer.py:19-292): same constructor keywords and
validation, same step(closure) contract, same per-parameter state keys.
Behind step() every parameter with a gradient is described in one table and
updated by four kernel launches per device (libturboadam_amd,
include/turboadam_amd.h), instead of the reference's per-parameter Python
loop.  Parameters must live on a HIP device; there is no CPU path.
"""

import ctypes
import math
import operator
import os

import numpy as np
import torch
from torch.optim import Optimizer

from . import _lib
from .costate import CoStateManager
from .oneq import init_v_state
from .utils import BLOCK_SIZE, num_blocks

# Key of the Philox4x32-10 stream that drives stochastic rounding.  The
# counter is (element/4, tensor_id, step, 0), so a step is reproducible from
# (seed, parameter order, step number) alone.
from .quantize import DEFAULT_SEED  # noqa: E402  (the Philox key of the stochastic rounding)

_DTYPES = {
    torch.float32: _lib.TAM_DTYPE_F32,
    torch.bfloat16: _lib.TAM_DTYPE_BF16,
    torch.float16: _lib.TAM_DTYPE_F16,
}

_F32 = ctypes.c_float


def _f32(x: float) -> float:
    """Round a Python float (double) to fp32, as torch does for a scalar operand."""
    return _F32(x).value


# numpy view of the descriptor layout (include/turboadam_amd.h TamTensor)
_DESC = np.dtype(_lib.TamTensor)
# the fields gathered per tensor, in the order _describe collects them
_ROW_FIELDS = ("param", "grad", "v_idx", "v_scales", "exp_avg_sq", "exp_avg", "signs", "labels", "norms", "amp",
               "alpha", "ef_residual", "n", "dtype", "flags", "v_bits", "tensor_id", "step", "k_lo", "k_hi")
# the fields a parameter group shares, in the order _group_fields returns them
_GROUP_FIELDS = ("c_wd", "beta1", "one_minus_beta1", "beta2", "one_minus_beta2", "bias_correction1",
                 "bias_correction2", "inv_bc2", "inv_bc2_f32", "eps", "neg_lr", "sqrt_block")
_SQRT_BLOCK_F32 = _f32(math.sqrt(BLOCK_SIZE))


_host_module = None


def _host():
    """The C++ host module of steady steps (csrc/tam_host.cpp, built by
    turboadam_amd.build); raises when it is missing."""
    global _host_module
    if _host_module is None:
        import importlib.machinery
        import importlib.util

        from .build import HOST_MODULE_PATH

        if not os.path.exists(HOST_MODULE_PATH):
            raise RuntimeError(f"turboadam_amd: host module not built ({HOST_MODULE_PATH}); "
                               "run turboadam_amd.build.build_library()")
        loader = importlib.machinery.ExtensionFileLoader("_tam_host", HOST_MODULE_PATH)
        spec = importlib.util.spec_from_loader("_tam_host", loader)
        mod = importlib.util.module_from_spec(spec)
        loader.exec_module(mod)
        _host_module = mod
    return _host_module


# byte offsets of the per-step fields a steady step rewrites in each descriptor row
_GRAD_OFF = _DESC.fields["grad"][1]
_STEP_OFF = _DESC.fields["step"][1]


def _row_tensors(state, compress_v: bool) -> tuple:
    """The state tensors a descriptor row points at, in a fixed order (None
    where a row has no such array).  A kept descriptor table is valid only
    while these are the same tensors: code that replaces one (a reset, an
    offload round trip) must make the next step rebuild its row."""
    if compress_v:
        cv = state["compressed_v"]
        v = (cv["indices"], cv["scales"])
    else:
        v = (state["exp_avg_sq"],)
    if state["_compress_m"]:
        mgr = state["m_mgr"]
        enc = mgr._encoded
        return v + (enc["sign_packed"], enc["labels"], enc["block_norms"], enc["scales"], mgr._alpha,
                    mgr._ef_residual)
    return v + (state["exp_avg"],)


def _tensor_ptrs(rows) -> list:
    """Device addresses of _row_tensors rows, flattened (0 for None)."""
    return [0 if t is None else t.data_ptr() for row in rows for t in row]


class _DeviceBuffers:
    """Per-device descriptor and workspace buffers, grown on demand, and the
    persistent pinned upload buffer of capturable steps."""

    def __init__(self, device):
        self.device = device
        self.desc = None
        self.ws = None
        self.pinned = None
        self.pinned_bytes = b""
        self.stream = None  # the stream of the last step that used these buffers
        self.captured = False  # a captured graph replays the descriptor upload from these buffers

    def fits(self, desc_bytes: int, ws_bytes: int, raw) -> bool:
        """Whether a step can run on these buffers without reallocating them or
        rewriting the pinned bytes a captured graph re-uploads (raw: the
        static descriptor bytes of a capturable step, or None)."""
        if self.desc is None or self.desc.numel() < desc_bytes or self.ws is None or self.ws.numel() < ws_bytes:
            return False
        return raw is None or raw == self.pinned_bytes

    def order_on(self, stream) -> None:
        """The buffers are reused from step to step, not reallocated: a step on
        another stream than the last one first waits for that stream's work.
        (torch.cuda.graph synchronises before a capture, so a capture needs no
        wait, and may not wait on a stream outside it.)"""
        if self.stream is not None and self.stream != stream and not torch.cuda.is_current_stream_capturing():
            stream.wait_stream(self.stream)
        self.stream = stream

    def upload_static(self, raw: bytes) -> torch.Tensor:
        """Pinned host copy of `raw` that a captured graph re-reads on every
        replay.  It is rewritten only when the descriptors change; a pending
        copy from it is waited for first (not possible during a capture)."""
        if raw != self.pinned_bytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("turboadam_amd: capturable step changed its tensors during graph capture; "
                                   "run an eager warm-up step with the same parameters and gradients first")
            if self.pinned is not None:
                torch.cuda.synchronize(self.device)  # a copy from it may be pending on any stream
            if self.pinned is None or self.pinned.numel() < len(raw):
                self.pinned = torch.empty(max(len(raw), 4096), dtype=torch.uint8, pin_memory=True)
            ctypes.memmove(self.pinned.data_ptr(), raw, len(raw))
            self.pinned_bytes = raw
        return self.pinned[: len(raw)]

    def desc_buffer(self, nbytes: int) -> torch.Tensor:
        if self.desc is None or self.desc.numel() < nbytes:
            self.desc = torch.empty(max(nbytes, 4096), dtype=torch.uint8, device=self.device)
        return self.desc

    def workspace(self, nbytes: int) -> torch.Tensor:
        if self.ws is None or self.ws.numel() < nbytes:
            self.ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=self.device)
        return self.ws


class _StepPlan:
    """The descriptor table of one device's step, kept from step to step while
    the same parameters have gradients and no state has been created,
    replaced or loaded since (TurboAdam._layout_version).  A later step
    rewrites only what changes between steps: gradient pointers, step numbers,
    the has-state flags and the group scalars (lr, betas, eps, weight decay,
    bias corrections)."""

    def __init__(self, key, table, gsel, groups, static_flags, costate, ef, capturable):
        self.key = key
        self.state_ptrs = None  # _tensor_ptrs of the rows' state tensors when the table was built
        self.row_cv = None      # compress_v of each row's group when the table was built
        self.table = table
        self.gsel = gsel              # group row of each descriptor row
        self.groups = groups          # (group, group_idx) of each group row
        self.static_flags = static_flags  # flags without HAS_STATE / HAS_EF / WD
        self.costate = costate        # rows with CoState m
        self.ef = ef                  # rows with error feedback
        self.capturable = capturable  # rows whose step fields the device fills
        self.any_capturable = bool(capturable.any())
        self.cost_rows = np.flatnonzero(costate)
        self.ef_rows = np.flatnonzero(ef)
        self.step_rows = np.flatnonzero(~capturable)


class _PinnedUpload:
    """Two pinned host buffers used in turn for the descriptor upload of eager
    steps; a buffer is rewritten only after the copy from it has completed."""

    def __init__(self):
        self.bufs = [None, None]
        self.events = [None, None]
        self.k = 0

    def stage(self, arr, nbytes: int) -> torch.Tensor:
        k = self.k = 1 - self.k
        if self.events[k] is not None:
            self.events[k].synchronize()
        if self.bufs[k] is None or self.bufs[k].numel() < nbytes:
            self.bufs[k] = torch.empty(max(nbytes, 4096), dtype=torch.uint8, pin_memory=True)
        ctypes.memmove(self.bufs[k].data_ptr(), ctypes.addressof(arr), nbytes)
        return self.bufs[k][:nbytes]

    def copied(self, stream) -> None:
        """Record that the copy from the buffer just staged is enqueued on stream."""
        ev = self.events[self.k]
        if ev is None:
            ev = self.events[self.k] = torch.cuda.Event()
        ev.record(stream)


class _FastStep:
    """The host side of a steady step, kept from the previous step: one device,
    no capturable group, the same parameters with gradients and unchanged state
    (TurboAdam._layout_version), every CoState tensor past its first update
    and every error-feedback residual written.  Such a step skips the
    per-parameter walk of _collect: the gradients are gathered by list
    comprehensions, checked only when a gradient object is new (dtype, layout,
    contiguity, device), the parameters' storage pointers are compared with the
    kept descriptor rows (p.data replaced: not steady), and the step numbers
    and bias corrections come from the kept state dicts.

    A step is not steady either when opt.state no longer holds the kept
    per-parameter dicts in the same order (cleared, an entry replaced or
    removed) or when a row's state tensors (_row_tensors) are not the kept
    objects; the full path then rebuilds what changed.  A state tensor is
    recognised by identity here; the full path compares device addresses."""

    def __init__(self, version, device, params, absent, rows, states, grads, pdtypes, bc_src, plan, state_map):
        self.version = version
        # the optimizer's state mapping and its per-parameter dicts, in order:
        # opt.state.clear(), opt.state[p] = {} or a new mapping is not steady
        self.state_map = state_map
        self.state_values = list(state_map.values())
        # the state tensors of each row (_row_tensors), by identity
        self.tensors = [t for st, cv in zip(states, plan.row_cv) for t in _row_tensors(st, cv)]
        self.device = device
        self.dev_index = device.index if device.index is not None else torch.cuda.current_device()
        self.params = params      # every parameter of the optimizer, in order
        self.absent = absent      # [p.grad is None] of the step this was built from
        self.rows = rows          # positions (in params) of the descriptor rows
        self.states = states      # their state dicts
        self.grads = grads        # the gradient objects last checked, per row
        self.pcodes = [_DTYPES[dt] for dt in pdtypes]  # their TAM_DTYPE_* codes
        self.bc_src = bc_src      # (bc key, group betas, state dict whose step sets the group's bias corrections)
        self.plan = plan
        self.row_params = [params[i] for i in rows]
        self.ptrs = [p.data_ptr() for p in self.row_params]  # parameter storage the descriptor rows point at


class TurboAdam(Optimizer):
    """Adam optimizer with compressed first and second moment storage.

    Args (reference optimizer.py:32-60):
        params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0,
        block_size=128, v_bits in {2,3,4,6,8} (default 4), compress_m=True,
        compress_v=True, null_pct=0.10, amp_pct=0.90, error_feedback=False,
        capturable=False, min_m_compress_elements=4096.

    philox_seed (keyword only, an addition): the 64-bit key of the Philox
    stream that drives stochastic rounding (attribute of the same name).
    """

    def __init__(
        self,
        params,
        lr: float = 1e-3,
        betas: tuple = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 0.0,
        block_size: int = 128,
        v_bits: int = 4,
        compress_m: bool = True,
        compress_v: bool = True,
        null_pct: float = 0.10,
        amp_pct: float = 0.90,
        error_feedback: bool = False,
        capturable: bool = False,
        min_m_compress_elements: int = 4096,
        *,
        philox_seed: int = DEFAULT_SEED,
    ):
        if v_bits not in (2, 3, 4, 6, 8):
            raise ValueError(f"v_bits must be one of {{2, 3, 4, 6, 8}}, got {v_bits}")
        defaults = dict(
            lr=lr,
            betas=betas,
            eps=eps,
            weight_decay=weight_decay,
            block_size=block_size,
            v_bits=v_bits,
            compress_m=compress_m,
            compress_v=compress_v,
            null_pct=null_pct,
            amp_pct=amp_pct,
            error_feedback=error_feedback,
            min_m_compress_elements=min_m_compress_elements,
            capturable=capturable,
        )
        super().__init__(params, defaults)
        self._group_step_tensors = {}
        self._found_inf = None
        self._keepalive = []  # states holding a contiguous copy of their gradient for this step
        if not 0 <= int(philox_seed) < (1 << 64):
            raise ValueError(f"philox_seed must be a 64-bit unsigned integer, got {philox_seed}")
        self.philox_seed = int(philox_seed)
        self._buffers = {}
        self._plans = {}
        self._uploads = {}
        # bumped whenever a state is created, replaced or loaded: a descriptor
        # table built before is then rebuilt (_StepPlan)
        self._layout_version = 0
        self._retired_buffers = []  # buffers a captured graph still replays
        self._skip_flags = {}
        self._bc_values = {}
        self._bc_tables = {}
        # Optional callable(pass_index, "begin"|"end") run around each of the four
        # launches (the step is then issued pass by pass); used to time kernels.
        self._pass_hook = None
        self._fast = None  # _FastStep of the last steady step

    def add_param_group(self, param_group):
        """torch.optim.Optimizer.add_param_group; later parameters' tensor ids
        (their positions in param_groups order) follow the new group's."""
        super().add_param_group(param_group)
        self._layout_version = getattr(self, "_layout_version", 0) + 1

    # ------------------------------------------------------------------
    # lazy state initialisation (reference optimizer.py:238-286)
    # ------------------------------------------------------------------
    def _init_state(self, p, group, group_idx, state):
        if p.device.type != "cuda":
            raise RuntimeError(
                f"turboadam_amd.TurboAdam steps parameters on an MI355X (HIP) device; got a parameter on {p.device}"
            )
        if p.numel() == 0:
            raise RuntimeError("turboadam_amd.TurboAdam: cannot optimise a parameter with no elements")
        block_size = group["block_size"]
        # capturable: the step counter lives on the device and the step advances it
        state["step"] = torch.zeros((), dtype=torch.int32, device=p.device) if group.get("capturable") else 0
        compress_this_m = group["compress_m"] and p.numel() >= group["min_m_compress_elements"]
        state["_compress_m"] = compress_this_m
        if compress_this_m:
            mgr = CoStateManager(
                block_size=block_size,
                null_pct=group["null_pct"],
                amp_pct=group["amp_pct"],
                error_feedback=group["error_feedback"],
            )
            mgr.allocate(p.numel(), p.device)
            state["m_mgr"] = mgr
        else:
            state["exp_avg"] = torch.zeros_like(p, dtype=torch.float32, memory_format=torch.contiguous_format)
        if not group["compress_v"]:
            state["exp_avg_sq"] = torch.zeros_like(p, dtype=torch.float32, memory_format=torch.contiguous_format)
        self._link_bias_tensors(p, group_idx, state)
        self._layout_version += 1

    def _link_bias_tensors(self, p, group_idx, state):
        device_key = (group_idx, p.device.type, p.device.index)
        if device_key not in self._group_step_tensors:
            self._group_step_tensors[device_key] = {
                "bc1": torch.empty(1, dtype=torch.float32, device=p.device),
                "bc2": torch.empty(1, dtype=torch.float32, device=p.device),
            }
        t = self._group_step_tensors[device_key]
        state["_bc1"] = t["bc1"]
        state["_bc2"] = t["bc2"]

    # ------------------------------------------------------------------
    # bias corrections (reference optimizer.py:172-188)
    # ------------------------------------------------------------------
    def _collect(self):
        """One pass over the parameters (reference optimizer.py:224-292).

        Parameters with a gradient get their lazy state and are grouped per
        device with their tensor ids (their position in the parameter list).
        The bias corrections of the coming step are computed per (group,
        device): the reference fills one shared 1-element tensor per (group,
        device) once per parameter in the group (optimizer.py:172-188), so the
        value every parameter uses is the one of the group's last parameter
        with state; that value is computed here and written to the shared
        tensors.  Step counters advance only once the step is launched.
        """
        per_device = {}
        self._bc_values = {}
        tid = -1
        for group_idx, group in enumerate(self.param_groups):
            device_step = group.get("capturable")  # computed on the device (tam_k_device_step)
            last = {}
            for p in group["params"]:
                tid += 1
                if p.grad is None:
                    state = self.state.get(p)
                    if state is None:
                        continue
                else:
                    state = self.state[p]
                    if len(state) == 0:
                        self._init_state(p, group, group_idx, state)
                    if group["compress_v"] and "compressed_v" not in state:
                        state["compressed_v"] = init_v_state(p, group["v_bits"], group["block_size"])
                        self._layout_version += 1
                    dev = p.device
                    items = per_device.get(dev)
                    if items is None:
                        items = per_device[dev] = []
                    items.append((p, state, group, group_idx, tid))
                if not device_step:
                    last[p.device] = state["step"]
            if last:
                beta1, beta2 = group["betas"]
                for dev, step in last.items():
                    next_step = step + 1
                    self._bc_values[(group_idx, dev.type, dev.index)] = (1.0 - beta1**next_step, 1.0 - beta2**next_step)
        for key, (bc1, bc2) in self._bc_values.items():
            t = self._group_step_tensors.get(key)
            if t is not None:
                t["bc1"].fill_(bc1)
                t["bc2"].fill_(bc2)
        return per_device

    # ------------------------------------------------------------------
    # state dict (reference optimizer.py:194-218)
    # ------------------------------------------------------------------
    _PACKED_V = {"indices": torch.uint8, "scales": torch.float16}
    _FP32_STATE = ("exp_avg", "exp_avg_sq")

    def state_dict(self):
        """torch's optimizer state dict plus the Philox key ("philox_seed"), so
        that a resumed run draws the same stochastic rounding."""
        for group in self.param_groups:
            if not group.get("capturable"):
                continue
            for p in group["params"]:  # a device-skipped first step leaves no encoding
                st = self.state.get(p, {})
                if st.get("_compress_m") and isinstance(st.get("step"), torch.Tensor):
                    st["m_mgr"]._has_state = int(st["step"]) > 0
        sd = super().state_dict()
        sd["philox_seed"] = self.philox_seed
        return sd

    @staticmethod
    def _adopt_manager(mgr, group) -> CoStateManager:
        """A CoStateManager of this package holding mgr's state.  mgr may be one
        loaded from a reference checkpoint (only the attributes the reference
        pickles, costate.py:357-365); settings it lacks come from the group."""
        new = CoStateManager(block_size=getattr(mgr, "block_size", group["block_size"]),
                             error_feedback=getattr(mgr, "_error_feedback", group["error_feedback"]),
                             null_pct=getattr(mgr, "_null_pct", group["null_pct"]),
                             amp_pct=getattr(mgr, "_amp_pct", group["amp_pct"]))
        for key in ("_has_state", "_alpha", "_encoded", "_original_numel", "_ef_residual"):
            if hasattr(mgr, key):
                setattr(new, key, getattr(mgr, key))
        return new

    def load_state_dict(self, state_dict):
        """Load optimizer state.

        torch's loader casts every state tensor to the parameter dtype (which
        would round the f16 v scales of a bf16 parameter to bf16).  The packed
        tensors are kept aside and restored unchanged, so a resumed run
        continues bit for bit; CoStateManager tensors are moved to the
        parameter's device as in the reference; a reference checkpoint's
        `rand_buf` is dropped (this implementation draws from Philox), and its
        CoStateManager objects are adopted into this package's class.  A
        "philox_seed" entry (written by state_dict) restores the Philox key.
        """
        self._layout_version += 1
        if "philox_seed" in state_dict:
            state_dict = dict(state_dict)
            self.philox_seed = int(state_dict.pop("philox_seed"))
        saved_v, saved_fp32 = {}, {}
        for pid, st in state_dict.get("state", {}).items():
            if not isinstance(st, dict):
                continue
            cv = st.get("compressed_v")
            if isinstance(cv, dict):
                saved_v[pid] = {k: cv[k] for k in self._PACKED_V if isinstance(cv.get(k), torch.Tensor)}
            # fp32 moments of a 16-bit parameter: torch's loader would round them to its dtype
            saved_fp32[pid] = {k: st[k] for k in self._FP32_STATE if isinstance(st.get(k), torch.Tensor)}
        # saved ids pair with the parameters in order, as torch's loader pairs them
        saved_ids = [i for g in state_dict.get("param_groups", []) for i in g["params"]]
        super().load_state_dict(state_dict)
        param_to_id = {id(p): i for i, p in zip(saved_ids, (p for g in self.param_groups for p in g["params"]))}
        for group_idx, group in enumerate(self.param_groups):
            for p in group["params"]:
                if p not in self.state:
                    continue
                state = self.state[p]
                device = p.device
                pid = param_to_id.get(id(p))
                step = state.get("step", 0)
                if group.get("capturable"):  # torch's loader makes it f32 on the device
                    state["step"] = torch.as_tensor(step).to(device=device, dtype=torch.int32).reshape(()).clone()
                else:
                    state["step"] = int(step.item()) if isinstance(step, torch.Tensor) else int(step)
                cv = state.get("compressed_v")
                if isinstance(cv, dict):
                    cv.pop("rand_buf", None)
                    for k, dt in self._PACKED_V.items():
                        src = saved_v.get(pid, {}).get(k, cv.get(k))
                        if isinstance(src, torch.Tensor):
                            cv[k] = src.to(device=device, dtype=dt).clone().contiguous()
                mgr = state.get("m_mgr")
                if mgr is not None:
                    mgr = state["m_mgr"] = self._adopt_manager(mgr, group)
                    if isinstance(mgr._alpha, torch.Tensor):
                        mgr._alpha = mgr._alpha.to(device=device, dtype=torch.float32).clone()
                    else:
                        mgr._alpha = torch.tensor(float(mgr._alpha), dtype=torch.float32, device=device)
                    if mgr._encoded is not None:
                        canon = {"labels": torch.uint8, "sign_packed": torch.uint8,
                                 "block_norms": torch.float32, "scales": torch.float16}
                        for key, dt in canon.items():
                            if key in mgr._encoded:
                                mgr._encoded[key] = mgr._encoded[key].to(device=device, dtype=dt).clone()
                    else:
                        mgr.allocate(p.numel(), device)
                    if mgr._ef_residual is not None:
                        mgr._ef_residual = mgr._ef_residual.to(device=device, dtype=torch.float32).clone() \
                            .contiguous().reshape(p.shape)
                for key in self._FP32_STATE:
                    if key in state:
                        src = saved_fp32.get(pid, {}).get(key, state[key])
                        state[key] = src.to(device=device, dtype=torch.float32).clone() \
                            .contiguous().reshape(p.shape)
                self._link_bias_tensors(p, group_idx, state)

    # ------------------------------------------------------------------
    # the step
    # ------------------------------------------------------------------
    def _group_fields(self, group, group_idx, device):
        """The descriptor fields one group shares on one device, each rounded
        to fp32 once (the kernels' scalars; reference optimizer.py:88-170)."""
        lr = group["lr"]
        beta1, beta2 = group["betas"]
        wd = group["weight_decay"]
        if group.get("capturable"):
            bc1 = bc2 = 1.0  # the first launch takes them from the device table
        else:
            bc1, bc2 = self._bc_values.get((group_idx, device.type, device.index), (1.0, 1.0))
        bc2_f = _f32(bc2)
        inv_bc2 = 1.0 / bc2_f
        return (_f32(1.0 - lr * wd), _f32(beta1), _f32(1.0 - beta1), _f32(beta2), _f32(1.0 - beta2), _f32(bc1),
                bc2_f, inv_bc2, _f32(inv_bc2), _f32(group["eps"]), _f32(-lr), _SQRT_BLOCK_F32)

    def _grad_ptr(self, p, state) -> int:
        """Device address of p's gradient (checked; a contiguous copy of a
        strided one is kept alive for the step)."""
        g = p.grad
        if g.is_sparse:
            raise RuntimeError("turboadam_amd.TurboAdam does not support sparse gradients")
        if g.dtype != p.dtype or g.device != p.device:
            raise RuntimeError("turboadam_amd: gradient dtype/device must match the parameter")
        if not g.is_contiguous():
            g = g.contiguous()
            state["_grad_keepalive"] = g
            self._keepalive.append(state)
        return g.data_ptr()

    def _describe(self, device, items) -> _StepPlan:
        """The descriptor table (TamTensor rows) of one device's step.

        The per-tensor fields are gathered in one pass over the items and
        written column by column; the scalars a group shares are computed
        once per group.  The derived fields stay zero for tam_prepare."""
        rows = []
        group_rows = []
        groups = {}
        group_list = []
        device_step = []
        for p, state, group, group_idx, tid in items:
            gi = groups.get(group_idx)
            if gi is None:
                if group["block_size"] != BLOCK_SIZE:
                    raise NotImplementedError("turboadam_amd kernels use 128-element blocks (block_size=128)")
                gi = groups[group_idx] = (len(group_rows), group["compress_v"], bool(group.get("capturable")))
                group_rows.append(self._group_fields(group, group_idx, device))
                group_list.append((group, group_idx))
            gk, compress_v, capturable = gi
            flags = 0
            code = _DTYPES.get(p.dtype)
            if code is None:
                raise NotImplementedError(f"turboadam_amd: unsupported parameter dtype {p.dtype}")
            if not p.is_contiguous():
                raise RuntimeError("turboadam_amd: parameters must be contiguous")
            gptr = self._grad_ptr(p, state)
            n = p.numel()
            nb = num_blocks(n)
            v_idx = v_scales = v_bits = exp_avg_sq = exp_avg = 0
            signs = labels = norms = amp = alpha = ef = 0
            k_lo = k_hi = 0
            if compress_v:
                cv = state["compressed_v"]
                idx, scl = cv["indices"], cv["scales"]
                if idx.dtype != torch.uint8 or scl.dtype != torch.float16:
                    raise RuntimeError("turboadam_amd: compressed_v tensors have unexpected dtypes")
                if idx.numel() != nb * BLOCK_SIZE or scl.numel() != nb * 2:
                    raise RuntimeError("turboadam_amd: compressed_v does not match the parameter size")
                flags |= _lib.TAM_FLAG_COMPRESS_V
                v_idx, v_scales, v_bits = idx.data_ptr(), scl.data_ptr(), cv["n_bits"]
            else:
                exp_avg_sq = state["exp_avg_sq"].data_ptr()
            if state["_compress_m"]:
                mgr = state["m_mgr"]
                enc = mgr._encoded
                flags |= _lib.TAM_FLAG_COSTATE
                if mgr._has_state:
                    flags |= _lib.TAM_FLAG_HAS_STATE
                signs = enc["sign_packed"].data_ptr()
                labels = enc["labels"].data_ptr()
                norms = enc["block_norms"].data_ptr()
                amp = enc["scales"].data_ptr()
                alpha = mgr._alpha.data_ptr()
                k_lo, k_hi = mgr.ranks(nb)
                if mgr._error_feedback:
                    # costate.py:409-437: the residual exists from the tensor's first
                    # update on; that update writes it without reading it
                    flags |= _lib.TAM_FLAG_EF
                    if mgr._ef_residual is None:
                        mgr._ef_residual = torch.zeros_like(p, dtype=torch.float32)
                        self._layout_version += 1
                    else:
                        flags |= _lib.TAM_FLAG_HAS_EF
                    ef = mgr._ef_residual.data_ptr()
            else:
                exp_avg = state["exp_avg"].data_ptr()
            if capturable:
                device_step.append((len(rows), p, state, group))
                step = 0  # filled on the device
            else:
                step = state["step"] + 1  # the counter advances once the step is launched
            rows.append((p.data_ptr(), gptr, v_idx, v_scales, exp_avg_sq, exp_avg, signs, labels, norms,
                         amp, alpha, ef, n, code, flags, v_bits, tid & 0xFFFFFFFF, step & 0xFFFFFFFF, k_lo, k_hi,
                         gk, capturable))
        table = np.zeros(len(rows), dtype=_DESC)
        cols = list(zip(*rows)) if rows else [()] * (len(_ROW_FIELDS) + 2)
        for name, col in zip(_ROW_FIELDS, cols):
            table[name] = col
        gsel = np.asarray(cols[-2], dtype=np.intp)
        capt = np.asarray(cols[-1], dtype=bool)
        plan = _StepPlan(None, table, gsel, group_list, None, (table["flags"] & _lib.TAM_FLAG_COSTATE) != 0,
                         (table["flags"] & _lib.TAM_FLAG_EF) != 0, capt)
        self._set_group_fields(plan, device, group_rows)
        if device_step:
            self._describe_device_step(table, device, device_step)
        plan.static_flags = table["flags"] & np.uint32(
            ~(_lib.TAM_FLAG_HAS_STATE | _lib.TAM_FLAG_HAS_EF | _lib.TAM_FLAG_WD) & 0xFFFFFFFF)
        plan.row_cv = [bool(group["compress_v"]) for _, _, group, _, _ in items]
        plan.state_ptrs = _tensor_ptrs(_row_tensors(it[1], cv) for it, cv in zip(items, plan.row_cv))
        return plan

    def _set_group_fields(self, plan, device, group_rows=None) -> None:
        """The fields a group shares (lr, betas, eps, weight decay and its flag,
        bias corrections), for every row."""
        if group_rows is None:
            group_rows = [self._group_fields(g, gi, device) for g, gi in plan.groups]
        if not group_rows:
            return
        t = plan.table
        gvals = np.asarray(group_rows, dtype=np.float64)
        for j, name in enumerate(_GROUP_FIELDS):
            t[name] = gvals[plan.gsel, j]
        wd = np.asarray([_lib.TAM_FLAG_WD if g["weight_decay"] != 0.0 else 0 for g, _ in plan.groups], np.uint32)
        t["flags"] = (t["flags"] & np.uint32(~_lib.TAM_FLAG_WD & 0xFFFFFFFF)) | wd[plan.gsel]

    def _refresh(self, plan, device, items) -> None:
        """Per-step fields of a kept descriptor table: gradient pointers, step
        numbers, has-state flags, group scalars (the rest is unchanged since
        the plan was built: the same parameters, the same state arrays)."""
        t = plan.table
        t["grad"] = [self._grad_ptr(p, state) for p, state, _, _, _ in items]
        if plan.step_rows.size:
            t["step"][plan.step_rows] = [(items[i][1]["step"] + 1) & 0xFFFFFFFF for i in plan.step_rows]
        flags = plan.static_flags.copy()
        host = ~plan.capturable  # capturable rows: the device sets HAS_STATE / HAS_EF
        if plan.cost_rows.size:
            hs = np.zeros(len(items), bool)
            hs[plan.cost_rows] = [items[i][1]["m_mgr"]._has_state for i in plan.cost_rows]
            flags[hs & host] |= np.uint32(_lib.TAM_FLAG_HAS_STATE)
        if plan.ef_rows.size:
            he = np.zeros(len(items), bool)
            he[plan.ef_rows] = True  # the residual exists (allocated when the plan was built) and has been written
            flags[he & host] |= np.uint32(_lib.TAM_FLAG_HAS_EF)
        t["flags"] = flags
        self._set_group_fields(plan, device)
        if plan.any_capturable:
            t["found_inf"][plan.capturable] = self._skip_ptr if self._found_inf is not None else 0

    # ------------------------------------------------------------------
    # capturable steps (the step counter and bias corrections on the device)
    # ------------------------------------------------------------------
    _BC_MAX_STEPS = 1 << 22

    def _bc_table(self, beta1: float, beta2: float, device):
        """fp32 (1 - beta1^t, 1 - beta2^t) for t = 1.. until both are exactly 1
        (they stay 1 after), computed as the reference does (Python floats,
        optimizer.py:172-188), as a device tensor."""
        key = (float(beta1), float(beta2), device)
        if key not in self._bc_tables:
            vals = []
            t = 0
            while True:
                t += 1
                b1, b2 = 1.0 - beta1**t, 1.0 - beta2**t
                vals += [b1, b2]
                if (_f32(b1) == 1.0 and _f32(b2) == 1.0) or t >= self._BC_MAX_STEPS:
                    break
            if _f32(vals[-2]) != 1.0 or _f32(vals[-1]) != 1.0:
                raise NotImplementedError(f"turboadam_amd: capturable with betas {beta1, beta2} needs bias "
                                          f"corrections beyond {self._BC_MAX_STEPS} steps")
            table = torch.tensor(vals, dtype=torch.float64).to(torch.float32).to(device)
            self._bc_tables[key] = (table, t)
        return self._bc_tables[key]

    def _describe_device_step(self, table, device, rows):
        """Fields of a capturable step: the kernels' first launch fills step,
        the bias corrections and the HAS_* flags from device counters, so the
        descriptor itself stays the same from step to step."""
        per_group = {}  # id(group) -> (bias-correction source pointer, table pointer, table length)
        idx, step_ptrs, cols = [], [], []
        for i, p, state, group in rows:
            step = state["step"]
            if not (isinstance(step, torch.Tensor) and step.dtype == torch.int32 and step.device == p.device):
                raise RuntimeError("turboadam_amd: a capturable parameter's state['step'] must be an int32 tensor "
                                   "on its device")
            g = per_group.get(id(group))
            if g is None:
                src = None  # the group's last parameter with state on this device (optimizer.py:172-188)
                for q in group["params"]:
                    if q in self.state and q.device == device:
                        src = self.state[q]["step"]
                beta1, beta2 = group["betas"]
                bc_table, bc_len = self._bc_table(beta1, beta2, device)
                g = per_group[id(group)] = (src.data_ptr(), bc_table.data_ptr(), bc_len)
            idx.append(i)
            step_ptrs.append(step.data_ptr())
            cols.append(g)
        sel = np.asarray(idx, dtype=np.intp)
        clear = np.uint32(_lib.TAM_FLAG_HAS_STATE | _lib.TAM_FLAG_HAS_EF)
        table["flags"][sel] = (table["flags"][sel] & ~clear) | np.uint32(_lib.TAM_FLAG_DEVICE_STEP)
        table["step_dev"][sel] = step_ptrs
        src_ptr, tab_ptr, tab_len = zip(*cols)
        table["bc_step"][sel] = src_ptr
        table["bc_table"][sel] = tab_ptr
        table["bc_len"][sel] = tab_len
        table["found_inf"][sel] = self._skip_ptr if self._found_inf is not None else 0

    def _skip_flag(self, device, found_inf: torch.Tensor) -> torch.Tensor:
        """A persistent per-device copy of GradScaler's found_inf (its tensor is
        new every step; the descriptors of a captured step keep one address)."""
        flag = self._skip_flags.get(device)
        if flag is None:
            flag = self._skip_flags[device] = torch.zeros(1, dtype=torch.float32, device=device)
        flag.copy_(found_inf.reshape(1))
        return flag

    def _device_buffers(self, device, capturing: bool) -> _DeviceBuffers:
        """The device's reusable buffers.  Buffers that a captured graph uses
        stay as they are for its replays: an eager step that would have to
        grow them or rewrite their pinned descriptor bytes moves to fresh
        buffers (_prepare_buffers), and the captured ones are kept alive."""
        bufs = self._buffers.get(device)
        if bufs is None:
            bufs = self._buffers[device] = _DeviceBuffers(device)
        if capturing:
            bufs.captured = True
        return bufs

    def _prepare_buffers(self, device, bufs, desc_bytes, ws_bytes, raw, capturing: bool) -> _DeviceBuffers:
        if bufs.captured and not capturing and not bufs.fits(desc_bytes, ws_bytes, raw):
            self._retired_buffers.append(bufs)
            bufs = self._buffers[device] = _DeviceBuffers(device)
            with torch.cuda.device(device):
                bufs.order_on(torch.cuda.current_stream(device))
        return bufs

    def _launch(self, device, items):
        lib = _lib.load()
        capturing = torch.cuda.is_current_stream_capturing()
        bufs = self._device_buffers(device, capturing)
        with torch.cuda.device(device):
            bufs.order_on(torch.cuda.current_stream(device))
            if self._found_inf is not None:
                self._skip_ptr = self._skip_flag(device, self._found_inf).data_ptr()
        # a parameter whose storage was replaced (p.data = ..., a dtype or
        # device change) needs its descriptor row rebuilt; so does a row whose
        # state tensors were replaced, and a capturable group whose betas
        # changed (its bias-correction table, _describe_device_step)
        key = (tuple(it[4] for it in items), tuple(it[0].data_ptr() for it in items),
               tuple(tuple(g["betas"]) for g in self.param_groups if g.get("capturable")))
        plan = self._plans.get(device)
        if plan is not None and plan.key == (key, self._layout_version):
            try:
                row_cv = [bool(it[2]["compress_v"]) for it in items]
                same = row_cv == plan.row_cv and _tensor_ptrs(
                    _row_tensors(it[1], cv) for it, cv in zip(items, row_cv)) == plan.state_ptrs
            except KeyError:
                same = False
            if not same:
                plan = None
        if plan is None or plan.key != (key, self._layout_version):
            plan = self._describe(device, items)
            plan.key = (key, self._layout_version)  # after _describe, which may create an EF residual
            self._plans[device] = plan
        else:
            self._refresh(plan, device, items)
        self._submit(lib, device, plan, bufs, capturing)
        for p, state, group, group_idx, tid in items:
            if not group.get("capturable"):
                state["step"] += 1  # capturable: the step's first launch counts it
            if state["_compress_m"]:
                mgr = state["m_mgr"]
                if not mgr._has_state:
                    mgr._has_state = True
                    mgr._original_numel = p.numel()
        return plan

    def _submit(self, lib, device, plan, bufs, capturing: bool) -> None:
        """Derived fields (tam_prepare), buffers, the descriptor upload and the
        step's launches on the device's current stream."""
        table = plan.table
        n = len(table)
        arr = (_lib.TamTensor * n).from_buffer(table)
        info = _lib.TamStepInfo()
        _lib.check(lib.tam_prepare(arr, n, ctypes.byref(info)), "tam_prepare")
        nbytes = ctypes.sizeof(arr)
        bufs = self._prepare_buffers(device, bufs, nbytes, info.ws_bytes, bytes(arr) if info.n_device_step else None,
                                     capturing)
        upload = None
        if info.n_device_step:
            # a captured graph replays this copy: the same pinned bytes every time
            host = bufs.upload_static(bytes(arr))
        else:
            upload = self._uploads.get(device)
            if upload is None:
                upload = self._uploads[device] = _PinnedUpload()
            host = upload.stage(arr, nbytes)
        desc = bufs.desc_buffer(nbytes)
        ws = bufs.workspace(info.ws_bytes)
        with torch.cuda.device(device):
            stream = torch.cuda.current_stream(device)
            desc[:nbytes].copy_(host, non_blocking=True)
            if upload is not None:
                upload.copied(stream)
            self._issue(lib, desc.data_ptr(), arr, info, ws, stream.cuda_stream)

    # ------------------------------------------------------------------
    # steady steps (_FastStep)
    # ------------------------------------------------------------------
    def _keep_fast(self, per_device, plans) -> None:
        """Keep what a following step with the same gradients needs (or drop
        it when this step's shape does not allow a fast one)."""
        self._fast = None
        if len(per_device) != 1 or self._keepalive:
            return
        (device, items), = per_device.items()
        if any(group.get("capturable") for group in self.param_groups):
            return
        for _, state, _, _, _ in items:
            if state["_compress_m"]:
                mgr = state["m_mgr"]
                if not mgr._has_state or (mgr._error_feedback and mgr._ef_residual is None):
                    return
        plan = plans[device]
        params = [p for group in self.param_groups for p in group["params"]]
        pos = {id(p): i for i, p in enumerate(params)}
        rows = [pos[id(p)] for p, _, _, _, _ in items]
        bc_src = []
        for group_idx, group in enumerate(self.param_groups):
            src = None  # the group's last parameter with state (optimizer.py:172-188)
            for q in group["params"]:
                st = self.state.get(q)
                if st is not None and q.device == device:
                    src = st
            if src is not None:
                bc_src.append(((group_idx, device.type, device.index), group, src))
        self._fast = _FastStep(self._layout_version, device, params, [p.grad is None for p in params], rows,
                               [it[1] for it in items], [it[0].grad for it in items], [it[0].dtype for it in items],
                               bc_src, plan, self.state)

    def _fast_state_kept(self, f) -> bool:
        """Whether opt.state still holds f's per-parameter dicts, in order, and
        each descriptor row's state tensors are the objects f kept."""
        st = self.state
        if st is not f.state_map or len(st) != len(f.state_values) or \
                not all(map(operator.is_, st.values(), f.state_values)):
            return False
        return _host().states_kept(f)

    def _fast_step(self) -> bool:
        """A steady step (_FastStep) if this one is; False (nothing done) otherwise."""
        f = self._fast
        if f is None or f.version != self._layout_version:
            return False
        st = self.state
        if st is not f.state_map or len(st) != len(f.state_values) or \
                not all(map(operator.is_, st.values(), f.state_values)):
            return False
        plan = f.plan
        if self._plans.get(f.device) is not plan:
            return False
        t = plan.table
        # per row, in C++: the same parameters with gradients, their dtypes and
        # storage, each new gradient's checks, the state tensors; then the
        # rows' gradient pointers and step numbers are written into t
        if not _host().steady_rows(f, t.ctypes.data, t.itemsize, _GRAD_OFF, _STEP_OFF):
            return False
        device = f.device
        self._bc_values = {}
        for key, group, src in f.bc_src:
            beta1, beta2 = group["betas"]
            next_step = src["step"] + 1
            bc = (1.0 - beta1**next_step, 1.0 - beta2**next_step)
            self._bc_values[key] = bc
            tb = self._group_step_tensors.get(key)
            if tb is not None:
                tb["bc1"].fill_(bc[0])
                tb["bc2"].fill_(bc[1])
        flags = plan.static_flags.copy()
        if plan.cost_rows.size:
            flags[plan.cost_rows] |= np.uint32(_lib.TAM_FLAG_HAS_STATE)
        if plan.ef_rows.size:
            flags[plan.ef_rows] |= np.uint32(_lib.TAM_FLAG_HAS_EF)
        t["flags"] = flags
        self._set_group_fields(plan, device)
        lib = _lib.load()
        bufs = self._device_buffers(device, False)
        with torch.cuda.device(device):
            bufs.order_on(torch.cuda.current_stream(device))
        self._submit(lib, device, plan, bufs, False)
        _host().advance_steps(f.states)
        return True

    def _issue(self, lib, desc_ptr: int, arr, info, ws: torch.Tensor, stream: int) -> None:
        """The step's launches: one tam_multi_tensor_step call, or the passes one
        by one around _pass_hook."""
        if self._pass_hook is None:
            rc = lib.tam_multi_tensor_step(desc_ptr, arr, ctypes.byref(info), self.philox_seed, ws.data_ptr(),
                                           ws.numel(), stream)
            _lib.check(rc, "tam_multi_tensor_step")
            return
        for k in range(5 if info.n_ef else 4):
            self._pass_hook(k, "begin")
            rc = lib.tam_step_pass(k, desc_ptr, ctypes.byref(info), self.philox_seed, ws.data_ptr(), ws.numel(),
                                   stream)
            _lib.check(rc, f"tam_step_pass({k})")
            self._pass_hook(k, "end")

    # GradScaler hands this optimizer grad_scale and found_inf (attributes set
    # around step()) instead of unscaling and checking on the host.
    _step_supports_amp_scaling = True

    def _unscale_grads(self, grad_scale: torch.Tensor) -> None:
        """Gradients times f32(1/scale), the op and rounding of GradScaler.unscale_."""
        inv = grad_scale.double().reciprocal().float()
        per = {}
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is not None:
                    per.setdefault((p.grad.device, p.grad.dtype), []).append(p.grad)
        for (device, _), grads in per.items():
            dummy = torch.zeros(1, dtype=torch.float32, device=device)
            torch._amp_foreach_non_finite_check_and_unscale_(grads, dummy, inv.to(device))

    @torch.no_grad()
    def step(self, closure=None):
        """Perform a single optimization step (reference optimizer.py:224-292).

        Under a GradScaler (torch.amp), the attributes grad_scale and found_inf
        are set: gradients are unscaled first, and the step is skipped when
        found_inf is nonzero -- on the device, without a host sync, when every
        group with gradients is capturable; otherwise after one host read of
        found_inf, as GradScaler itself does for other optimizers."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        grad_scale = getattr(self, "grad_scale", None)
        found_inf = getattr(self, "found_inf", None)
        self._found_inf = None
        if found_inf is not None:
            active = [g for g in self.param_groups if any(p.grad is not None for p in g["params"])]
            if active and all(g.get("capturable") for g in active):
                if found_inf.dtype != torch.float32 or found_inf.numel() != 1:
                    raise RuntimeError("turboadam_amd: found_inf must be a one-element float32 tensor")
                self._found_inf = found_inf
            elif float(found_inf) != 0.0:
                return loss
        if grad_scale is not None:
            self._unscale_grads(grad_scale)
        elif found_inf is None and not torch.cuda.is_current_stream_capturing() and self._fast_step():
            return loss
        try:
            # one fused step of every parameter with a gradient (reference optimizer.py:88-170)
            per_device = self._collect()
            plans = {device: self._launch(device, items) for device, items in per_device.items()}
            if grad_scale is None and found_inf is None:
                self._keep_fast(per_device, plans)
            else:
                self._fast = None
        finally:
            self._found_inf = None
            for state in self._keepalive:
                state.pop("_grad_keepalive", None)
            self._keepalive = []
        return loss
