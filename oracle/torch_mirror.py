"""TEST INFRASTRUCTURE ONLY -- a torch-CPU restatement of the reference step.

Restates the reference CPU path (davidkny22/turboadam src/turboadam:
optimizer.py:88-292, costate.py:22-464, quantize.py:222-299, oneq.py:13-48)
with torch tensor operations in the same order, so that in "faithful" mode it
performs the same floating-point operations as the reference and reproduces
its outputs bit for bit (tests/golden fixtures pin this).  In "exact" mode
five library-defined operations are replaced by their exactly specified
counterparts -- the definition the C oracle and the GPU implement:

    exp, log         correctly rounded (64-bit-significand evaluation, one rounding)
    sqrt             correctly rounded (IEEE fp32)
    dot (alpha)      per 8 consecutive elements an fp32 pairwise tree of the
                     products (first level fused: fma(x0, y0, fl(x1*y1))),
                     widened to fp64; balanced fp64 pairwise tree over the 16
                     of a 128-element block, then over the blocks zero-padded
                     to a power of two, rounded once
    block L2 norms   the same per-block sums of squares, fp64 sqrt, rounded once

It also serves as the timed CPU baseline (faithful mode = the reference's
own CPU cost) and drives the per-step tie analysis of tests/test_golden.py.
Parameters are torch CPU tensors; state layout follows the reference.
"""

import math

import numpy as np
import torch

from . import oracle as O

BS = 128


# ---------------------------------------------------------------- op sets
class FaithfulOps:
    name = "faithful"

    @staticmethod
    def exp(x):
        return x.exp()

    @staticmethod
    def log(x):
        return x.log()

    @staticmethod
    def sqrt(x):
        return x.sqrt()

    @staticmethod
    def dot(a, b):
        return a.dot(b)

    @staticmethod
    def row_norms(x2d):
        return x2d.norm(dim=1)


def _pairwise_rows(x: np.ndarray) -> np.ndarray:
    """Balanced adjacent-pairwise sum of each row (row length a power of two)."""
    while x.shape[1] > 1:
        x = x.reshape(x.shape[0], x.shape[1] // 2, 2).sum(axis=2)
    return x[:, 0]


def _pairwise_pad(x: np.ndarray) -> float:
    P = 1
    while P < x.size:
        P <<= 1
    buf = np.zeros(P)
    buf[: x.size] = x
    return float(_pairwise_rows(buf.reshape(1, P))[0])


def _fma32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """fl32(a*b + c) of fp32 arrays with a single rounding (an fp32 fma).

    a*b is exact in fp64; TwoSum gives p + c = s + e exactly; s rounds to fp32
    once, except where s is an fp32 midpoint and e != 0, where e decides."""
    p = a.astype(np.float64) * b.astype(np.float64)
    c64 = c.astype(np.float64)
    s = p + c64
    bb = s - p
    e = (p - (s - bb)) + (c64 - bb)
    r = s.astype(np.float32)
    up = np.nextafter(r, np.float32(np.inf))
    dn = np.nextafter(r, np.float32(-np.inf))
    nxt = np.where(e > 0, up, dn)
    mid = (r.astype(np.float64) + nxt.astype(np.float64)) * 0.5
    fix = (e != 0) & (s == mid)
    return np.where(fix, nxt, r)


def _lane_partials(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """fp32 partials of 8 consecutive products (x, y: fp32 (rows, 8)):
    p_k = fma(x_2k, y_2k, fl(x_2k+1 * y_2k+1)), then (p0 + p1) + (p2 + p3)."""
    p = [_fma32(x[:, 2 * k], y[:, 2 * k], x[:, 2 * k + 1] * y[:, 2 * k + 1]) for k in range(4)]
    return (p[0] + p[1]) + (p[2] + p[3])


def _block_sums(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """Per 128-element block of fp32 (nb, 128) arrays: fp64 pairwise sum of the
    16 lane partials."""
    nb = x.shape[0]
    lanes = _lane_partials(x.reshape(nb * 16, 8), y.reshape(nb * 16, 8)).astype(np.float64)
    return _pairwise_rows(lanes.reshape(nb, 16))


class ExactOps:
    name = "exact"

    @staticmethod
    def exp(x):
        y = np.exp(x.numpy().astype(np.longdouble)).astype(np.float32)
        return torch.from_numpy(y)

    @staticmethod
    def log(x):
        with np.errstate(divide="ignore", invalid="ignore"):
            y = np.log(x.numpy().astype(np.longdouble)).astype(np.float32)
        return torch.from_numpy(y)

    @staticmethod
    def sqrt(x):
        return torch.from_numpy(np.sqrt(x.numpy()))

    @staticmethod
    def dot(a, b):
        n = a.numel()
        nb = (n + BS - 1) // BS
        x = np.zeros(nb * BS, np.float32)
        y = np.zeros(nb * BS, np.float32)
        x[:n] = a.numpy()
        y[:n] = b.numpy()
        blocks = _block_sums(x.reshape(nb, BS), y.reshape(nb, BS))
        return torch.tensor(np.float32(_pairwise_pad(blocks) + 0.0))

    @staticmethod
    def row_norms(x2d):
        x = np.ascontiguousarray(x2d.numpy(), dtype=np.float32)
        return torch.from_numpy(np.sqrt(_block_sums(x, x)).astype(np.float32))


# ---------------------------------------------------------------- helpers
def _pad(t: torch.Tensor, value=0.0):
    n = t.shape[0]
    r = n % BS
    if r == 0:
        return t
    return torch.cat([t, t.new_full((BS - r,), value)])


def pack_signs(values: torch.Tensor) -> torch.Tensor:
    """Sign bits (1 = negative), element 8j+k in byte j bit 7-k (costate.py:157-182)."""
    n = values.shape[0]
    extra = (8 - n % 8) % 8
    if extra:
        values = torch.cat([values, values.new_zeros(extra)])
    bits = (values < 0).to(torch.uint8).reshape(-1, 8)
    out = torch.zeros(bits.shape[0], dtype=torch.uint8)
    for k in range(8):
        out |= bits[:, k] << (7 - k)
    return out


def unpack_signs(packed: torch.Tensor, n: int) -> torch.Tensor:
    """+1 / -1 per element (costate.py:185-210)."""
    p = packed.to(torch.int32)
    sh = torch.arange(7, -1, -1, dtype=torch.int32)
    bits = ((p.unsqueeze(1) >> sh.unsqueeze(0)) & 1).float().reshape(-1)[:n]
    return 1.0 - 2.0 * bits


# ---------------------------------------------------------------- CoState
def costate_decode(enc, alpha, g, n):
    """m_hat = alpha*g + scale*sign (costate.py:261-324)."""
    labels = enc["labels"].to(torch.uint8)
    norms = enc["block_norms"].float()
    amp = enc["scales"].float()
    nb = labels.shape[0]
    signs = _pad(unpack_signs(enc["sign_packed"], n)).reshape(nb, BS)
    phase = norms / math.sqrt(BS)
    s = torch.zeros_like(phase)
    s[labels == 1] = phase[labels == 1]
    s[labels == 2] = amp[labels == 2]
    dh = (s.unsqueeze(1) * signs).reshape(-1)[:n]
    return alpha * g + dh


def costate_update(st, g, beta1, null_pct, amp_pct, ops, trace=None, ef=False):
    """CoStateManager.update (costate.py:367-464); st is updated.  With error
    feedback (ef, :409-437) the residual st["ef"] is added to g in the EMA
    (decompose keeps g) and, after encoding, updated with the encoding loss
    delta - decode(new encoding, alpha=0) (its EMA from the second step on)."""
    g = g.reshape(-1).float()
    n = g.numel()
    nb = (n + BS - 1) // BS
    m_hat = costate_decode(st, st["alpha"], g, n) if st["has_state"] else torch.zeros_like(g)
    g_corrected = g + st["ef"] if ef and st.get("ef") is not None else g
    m = beta1 * m_hat + (1.0 - beta1) * g_corrected
    gg = ops.dot(g, g)
    mg = ops.dot(m, g)
    alpha = torch.where(gg > 0, mg / gg, gg.new_zeros(()))
    delta = m - alpha * g
    dn = ops.row_norms(_pad(delta).reshape(nb, BS))
    mn = ops.row_norms(_pad(m).reshape(nb, BS))
    safe = mn.clone()
    safe[safe == 0.0] = 1.0
    r = dn / safe
    r[mn == 0.0] = 0.0
    srt = r.sort().values
    lo = max(0, int(null_pct * nb) - 1)
    hi = min(nb - 1, int(amp_pct * nb))
    t0, t1 = srt[lo], srt[hi]
    labels = torch.zeros(nb, dtype=torch.uint8)
    labels[r >= t0] = 1
    labels[r >= t1] = 2
    st["labels"] = labels
    st["sign_packed"] = pack_signs(delta)
    st["block_norms"] = dn.float()
    st["scales"] = (dn / math.sqrt(BS)).to(torch.float16)
    st["alpha"] = alpha.clone()
    st["has_state"] = True
    if ef:
        delta_hat = costate_decode(st, g.new_zeros(1), g, n)
        ef_error = delta - delta_hat
        st["ef"] = ef_error if st.get("ef") is None else beta1 * st["ef"] + (1.0 - beta1) * ef_error
    if trace is not None:
        trace.update(m=m, delta=delta, alpha=alpha, ratios=r, tau=(t0, t1), dn=dn, mn=mn)
    return m


# ---------------------------------------------------------------- 1Q
def v_update(cv, grad, beta2, uniforms, ops, trace=None):
    """fused_v_update (quantize.py:222-299); cv["indices"], cv["scales"] replaced."""
    idx, scales = cv["indices"], cv["scales"]
    n = cv["original_length"]
    nb = scales.shape[0]
    nbk = 2 ** cv["n_bits"]
    q = idx.to(torch.long).reshape(nb, BS)
    lmin = scales[:, 0].float().unsqueeze(1)
    lmax = scales[:, 1].float().unsqueeze(1)
    span = lmax - lmin
    v = ops.exp(lmin + (q.float() + 0.5) / nbk * span)
    gf = grad.reshape(-1).float()
    g2 = torch.zeros(nb * BS)
    g2[:n] = gf * gf
    v.mul_(beta2).add_(g2.reshape(nb, BS), alpha=1.0 - beta2)
    lg = ops.log(v.clamp(min=1e-38))
    valid = (torch.arange(nb).unsqueeze(1) * BS + torch.arange(BS).unsqueeze(0)) < n
    nmin = lg.masked_fill(~valid, float("inf")).min(dim=1).values
    nmax = lg.masked_fill(~valid, float("-inf")).max(dim=1).values
    cv["scales"] = torch.stack([nmin, nmax], dim=1).to(torch.float16)
    sp = (nmax - nmin).unsqueeze(1).clamp(min=1e-10)
    c = (lg - nmin.unsqueeze(1)) / sp * nbk
    f = c.floor()
    fr = c - f
    u = uniforms.reshape(nb, BS)
    cv["indices"] = (f + (u < fr).float()).clamp(0, nbk - 1).to(torch.uint8).reshape(-1)
    if trace is not None:
        trace.update(v=v, lg=lg, c=c, u=u, lmin=nmin, lmax=nmax)
    return v.reshape(-1)[:n]


def init_v(p, n_bits):
    """compress_v_logscale(full_like(p, 1e-30)) (oneq.py:13-48), a closed form: indices 0."""
    n = p.numel()
    nb = (n + BS - 1) // BS
    s = torch.tensor(1e-30, dtype=torch.float32).clamp(min=1e-38).log().to(torch.float16)
    return {"indices": torch.zeros(nb * BS, dtype=torch.uint8), "scales": s.repeat(nb, 2),
            "n_bits": n_bits, "original_shape": p.shape, "original_length": n, "block_size": BS}


# ---------------------------------------------------------------- optimizer
DEFAULTS = O.DEFAULTS


class MirrorTurboAdam:
    """Host logic of the reference optimizer over torch CPU parameters.

    params: a list of tensors, or a list of groups {"params": [...], **hyperparameters}
    (optimizer.py:224-292 over torch.optim's param_groups); add_param_group adds one."""

    def __init__(self, params, ops=FaithfulOps, seed=0, **kw):
        self.defaults = dict(DEFAULTS)
        self.defaults.update(kw)
        self.params = []
        self.param_groups = []
        self.ops = ops
        self.seed = seed
        self.state = {}
        groups = params if params and isinstance(params[0], dict) else [{"params": list(params)}]
        for g in groups:
            self.add_param_group(g)

    @property
    def group(self):
        return self.param_groups[0]

    def add_param_group(self, group):
        """torch.optim.Optimizer.add_param_group: unset hyperparameters are the
        defaults; the group's parameters follow all earlier ones."""
        grp = dict(self.defaults)
        grp.update({k: v for k, v in group.items() if k != "params"})
        start = len(self.params)
        self.params.extend(group["params"])
        grp["idx"] = list(range(start, len(self.params)))
        self.param_groups.append(grp)

    def init_state(self, i, p, grp):
        st = {"step": 0, "_compress_m": bool(grp["compress_m"] and p.numel() >= grp["min_m_compress_elements"])}
        if st["_compress_m"]:
            st["cs"] = {"has_state": False, "alpha": torch.tensor(0.0)}
        else:
            st["exp_avg"] = torch.zeros(p.numel(), dtype=torch.float32)
        if not grp["compress_v"]:
            st["exp_avg_sq"] = torch.zeros(p.numel(), dtype=torch.float32)
        else:
            st["compressed_v"] = init_v(p, grp["v_bits"])
        self.state[i] = st

    def step(self, grads, ops=None, traces=None):
        """grads: aligned with the flat parameter list (None = no gradient)."""
        ops = ops or self.ops
        for grp in self.param_groups:  # lazy state (optimizer.py:238-286)
            for i in grp["idx"]:
                if grads[i] is not None and i not in self.state:
                    self.init_state(i, self.params[i], grp)
        for grp in self.param_groups:
            with_state = [i for i in grp["idx"] if i in self.state]
            if not with_state:
                continue
            lr, (b1, b2), eps, wd = grp["lr"], grp["betas"], grp["eps"], grp["weight_decay"]
            # bias corrections from the group's last parameter with state (optimizer.py:172-188)
            last = self.state[with_state[-1]]["step"] + 1
            bc1 = torch.tensor([1.0 - b1**last], dtype=torch.float32)
            bc2 = torch.tensor([1.0 - b2**last], dtype=torch.float32)
            for i in grp["idx"]:
                g = grads[i]
                if g is None:
                    continue
                p = self.params[i]
                st = self.state[i]
                st["step"] += 1
                tr = {} if traces is not None else None
                if wd != 0.0:
                    p.mul_(1.0 - lr * wd)
                if st["_compress_m"]:
                    m = costate_update(st["cs"], g, b1, grp["null_pct"], grp["amp_pct"], ops, tr,
                                       ef=grp["error_feedback"]).reshape(p.shape)
                else:
                    st["exp_avg"].mul_(b1).add_(g.reshape(-1), alpha=1.0 - b1)
                    m = st["exp_avg"].reshape(p.shape)
                if grp["compress_v"]:
                    cv = st["compressed_v"]
                    nb = cv["scales"].shape[0]
                    u = torch.from_numpy(O.philox_uniforms(i, st["step"], self.seed, nb * BS))
                    v = v_update(cv, g, b2, u, ops, tr).reshape(p.shape)
                else:
                    v = st["exp_avg_sq"]
                    v.mul_(b2).addcmul_(g.reshape(-1), g.reshape(-1), value=1.0 - b2)
                    v = v.reshape(p.shape)
                denom = ops.sqrt(v / bc2).add_(eps)
                p.addcdiv_(m, denom * bc1, value=-lr)
                if traces is not None:
                    tr["denom"] = denom
                    traces[i] = tr

    def arrays(self, i) -> dict:
        """State of parameter i in the oracle's naming (numpy)."""
        st = self.state[i]
        out = {}
        if "compressed_v" in st:
            out["indices"] = st["compressed_v"]["indices"].numpy().copy()
            out["scales"] = st["compressed_v"]["scales"].reshape(-1).view(torch.int16).numpy().view(np.uint16).copy()
        if st["_compress_m"] and st["cs"]["has_state"]:
            cs = st["cs"]
            out["labels"] = cs["labels"].numpy().copy()
            out["sign_packed"] = cs["sign_packed"].numpy().copy()
            out["block_norms"] = cs["block_norms"].numpy().copy()
            out["amp"] = cs["scales"].view(torch.int16).numpy().view(np.uint16).copy()
            out["alpha"] = cs["alpha"].reshape(1).float().numpy().copy()
            if cs.get("ef") is not None:
                out["ef_residual"] = cs["ef"].numpy().copy()
        if "exp_avg" in st:
            out["exp_avg"] = st["exp_avg"].numpy().copy()
        if "exp_avg_sq" in st:
            out["exp_avg_sq"] = st["exp_avg_sq"].numpy().copy()
        return out
