"""CoState first-moment codec (reference src/turboadam/costate.py).

m = alpha*g + delta is stored as one fp32 alpha per tensor plus, per
128-element block, a label (0 null, 1 phase, 2 amplitude), the residual L2
norm (fp32), an fp16 amplitude scale and one sign bit per element (MSB first).

TurboAdam.step runs the whole update fused in its multi-tensor launches.
The reference's public functions are also available one tensor at a time,
with the same names and argument meaning, on the gfx950 kernels (the
step's arithmetic: fp32 lane partials and fp64 pairwise sums for the dot
products and block norms, exact radix selection).  Inputs must be on an
MI355X (HIP) device.
"""

import torch

from . import _lib
from .utils import BLOCK_SIZE, num_blocks


def _require_gpu(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"turboadam_amd.{what}: tensors must be on an MI355X (HIP) device, got {t.device}")


def _require_block_size(block_size: int) -> None:
    if block_size != BLOCK_SIZE:
        raise NotImplementedError("turboadam_amd supports block_size=128 only")


def _f32_flat(t: torch.Tensor) -> torch.Tensor:
    return t.reshape(-1).float().contiguous()


def _scalar_on(x, device) -> torch.Tensor:
    """A 1-element fp32 device tensor holding x (a Python number or a tensor)."""
    if isinstance(x, torch.Tensor):
        return x.reshape(1).to(device=device, dtype=torch.float32).contiguous()
    return torch.tensor([float(x)], dtype=torch.float32, device=device)


def decompose(m: torch.Tensor, g: torch.Tensor):
    """alpha = (m.g)/(g.g) (0 when g.g == 0) and delta = m - alpha*g
    (reference costate.py:22-43).  Returns (alpha 0-dim fp32, delta like m)."""
    _require_gpu(m, "decompose")
    lib = _lib.load()
    mf, gf = _f32_flat(m), _f32_flat(g)
    n = mf.numel()
    alpha = torch.empty(1, dtype=torch.float32, device=m.device)
    delta = torch.empty(n, dtype=torch.float32, device=m.device)
    ws = torch.empty(lib.tam_decompose_workspace(max(n, 1)), dtype=torch.uint8, device=m.device)
    with torch.cuda.device(m.device):
        _lib.check(lib.tam_decompose(mf.data_ptr(), gf.data_ptr(), n, alpha.data_ptr(), delta.data_ptr(),
                                     ws.data_ptr(), ws.numel(), _lib.stream_of(m.device)), "tam_decompose")
    return alpha.reshape(()), delta.reshape(m.shape)


def compute_block_ratios(delta: torch.Tensor, m: torch.Tensor, block_size: int = BLOCK_SIZE) -> torch.Tensor:
    """r_b = ||delta_b|| / ||m_b||, 0 where ||m_b|| == 0 (reference costate.py:51-86)."""
    _require_gpu(delta, "compute_block_ratios")
    _require_block_size(block_size)
    lib = _lib.load()
    df, mf = _f32_flat(delta), _f32_flat(m)
    n = df.numel()
    ratios = torch.empty(num_blocks(n), dtype=torch.float32, device=delta.device)
    with torch.cuda.device(delta.device):
        _lib.check(lib.tam_block_ratios(df.data_ptr(), mf.data_ptr(), n, ratios.data_ptr(),
                                        _lib.stream_of(delta.device)), "tam_block_ratios")
    return ratios


def threshold_ranks(nb: int, null_pct: float, amp_pct: float):
    """Sorted positions of the two thresholds (costate.py:115-117, Python double arithmetic)."""
    return max(0, int(null_pct * nb) - 1), min(nb - 1, int(amp_pct * nb))


def compute_thresholds(ratios: torch.Tensor, null_pct: float = 0.10, amp_pct: float = 0.90):
    """(tau0, tau1): the ratios at sorted positions max(0, int(null_pct*nb)-1) and
    min(nb-1, int(amp_pct*nb)), NaN sorting last (reference costate.py:94-118)."""
    _require_gpu(ratios, "compute_thresholds")
    lib = _lib.load()
    r = ratios.reshape(-1).float().contiguous()
    if r.data_ptr() % 16:
        r = r.clone()
    nb = r.numel()
    if nb == 0:
        raise IndexError("compute_thresholds: empty ratios")
    k_lo, k_hi = threshold_ranks(nb, null_pct, amp_pct)
    taus = torch.empty(2, dtype=torch.float32, device=r.device)
    ws = torch.empty(lib.tam_thresholds_workspace(nb), dtype=torch.uint8, device=r.device)
    with torch.cuda.device(r.device):
        _lib.check(lib.tam_thresholds(r.data_ptr(), nb, k_lo, k_hi, taus.data_ptr(), ws.data_ptr(), ws.numel(),
                                      _lib.stream_of(r.device)), "tam_thresholds")
    return taus[0], taus[1]


def classify_blocks(ratios: torch.Tensor, tau0, tau1) -> torch.Tensor:
    """label = 2 if r >= tau1, 1 if r >= tau0, else 0 (reference costate.py:126-149)."""
    _require_gpu(ratios, "classify_blocks")
    lib = _lib.load()
    r = ratios.reshape(-1).float().contiguous()
    taus = torch.cat([_scalar_on(tau0, r.device), _scalar_on(tau1, r.device)])
    labels = torch.empty(r.numel(), dtype=torch.uint8, device=r.device)
    with torch.cuda.device(r.device):
        _lib.check(lib.tam_classify(r.data_ptr(), r.numel(), taus.data_ptr(), labels.data_ptr(),
                                    _lib.stream_of(r.device)), "tam_classify")
    return labels


def encode_blocks(delta: torch.Tensor, labels: torch.Tensor, block_size: int = BLOCK_SIZE) -> dict:
    """Block norms, fp16 amplitudes and packed sign bits of delta; labels pass
    through (reference costate.py:213-258)."""
    _require_gpu(delta, "encode_blocks")
    _require_block_size(block_size)
    lib = _lib.load()
    df = _f32_flat(delta)
    n = df.numel()
    nb = num_blocks(n)
    dev = delta.device
    signs = torch.empty((n + 7) // 8, dtype=torch.uint8, device=dev)
    norms = torch.empty(nb, dtype=torch.float32, device=dev)
    amp = torch.empty(nb, dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        _lib.check(lib.tam_costate_encode(df.data_ptr(), n, signs.data_ptr(), norms.data_ptr(), amp.data_ptr(),
                                          _lib.stream_of(dev)), "tam_costate_encode")
    return {"labels": labels, "sign_packed": signs, "block_norms": norms, "scales": amp}


def _decode(encoded: dict, alpha, g: torch.Tensor, n: int, has_state: bool, ema: bool, beta1: float = 0.0):
    lib = _lib.load()
    dev = g.device
    gf = g.reshape(-1)
    if gf.dtype not in _lib.DTYPES:
        gf = gf.float()
    gf = gf.contiguous()
    if n != gf.numel():
        raise ValueError(f"decode_blocks: original_numel {n} does not match the gradient's {gf.numel()} elements")
    out = torch.empty(n, dtype=torch.float32, device=dev)
    ptrs = [0, 0, 0, 0, 0]
    keep = []
    if has_state:
        nb = num_blocks(n)
        if (encoded["labels"].numel() != nb or encoded["block_norms"].numel() != nb
                or encoded["scales"].numel() != nb or encoded["sign_packed"].numel() < (n + 7) // 8):
            raise ValueError(f"decode_blocks: the encoding does not cover {n} elements ({nb} blocks)")
        labels = encoded["labels"].to(device=dev, dtype=torch.uint8).contiguous()
        signs = encoded["sign_packed"].to(device=dev, dtype=torch.uint8).contiguous()
        norms = encoded["block_norms"].to(device=dev, dtype=torch.float32).contiguous()
        amp = encoded["scales"].to(device=dev, dtype=torch.float16).contiguous()
        a = _scalar_on(alpha, dev)
        keep = [labels, signs, norms, amp, a]
        ptrs = [t.data_ptr() for t in keep]
    b1 = float(torch.tensor(beta1, dtype=torch.float32))
    ob1 = float(torch.tensor(1.0 - beta1, dtype=torch.float32))
    with torch.cuda.device(dev):
        _lib.check(lib.tam_costate_decode(ptrs[0], ptrs[1], ptrs[2], ptrs[3], ptrs[4], gf.data_ptr(),
                                          _lib.DTYPES[gf.dtype], n, int(has_state), int(ema), b1, ob1,
                                          out.data_ptr(), _lib.stream_of(dev)), "tam_costate_decode")
    del keep
    return out


def decode_blocks(encoded: dict, alpha, g: torch.Tensor, block_size: int = BLOCK_SIZE,
                  original_numel: int = None) -> torch.Tensor:
    """m_hat = alpha*g + s_b*sign (s_b: 0, norm_b/sqrt(128) or the fp16
    amplitude by label), in fp32 with the shape of g (reference costate.py:261-324)."""
    _require_gpu(g, "decode_blocks")
    _require_block_size(block_size)
    n = g.numel() if original_numel is None else original_numel
    return _decode(encoded, alpha, g, n, True, False).reshape(g.shape)


class CoStateManager:
    """Per-tensor CoState state (same attributes as the reference, costate.py:332-365).

    TurboAdam keeps one per CoState parameter and updates it inside the fused
    step; update() runs the reference's per-tensor procedure on its own.
    """

    def __init__(self, block_size: int = BLOCK_SIZE, error_feedback: bool = False, null_pct: float = 0.10,
                 amp_pct: float = 0.90) -> None:
        self.block_size = block_size
        self._null_pct = null_pct
        self._amp_pct = amp_pct
        self._has_state = False
        self._alpha = 0.0
        self._encoded = None
        self._original_numel = 0
        self._error_feedback = error_feedback
        self._ef_residual = None

    def allocate(self, numel: int, device: torch.device) -> None:
        """Create the persistent device buffers (the reference clones them on its first update, :441-451)."""
        nb = num_blocks(numel, self.block_size)
        self._alpha = torch.zeros((), dtype=torch.float32, device=device)
        self._encoded = {
            "labels": torch.zeros(nb, dtype=torch.uint8, device=device),
            "sign_packed": torch.zeros((numel + 7) // 8, dtype=torch.uint8, device=device),
            "block_norms": torch.zeros(nb, dtype=torch.float32, device=device),
            "scales": torch.zeros(nb, dtype=torch.float16, device=device),
        }

    def ranks(self, nb: int):
        """Sorted positions of the two thresholds (costate.py:115-117)."""
        return threshold_ranks(nb, self._null_pct, self._amp_pct)

    def update(self, g: torch.Tensor, beta1: float) -> torch.Tensor:
        """One CoState step for gradient g (reference costate.py:367-464): decode
        the previous state (or zeros), m = beta1*m_hat + (1-beta1)*g, then
        decompose, ratios, thresholds, labels and encode into the persistent
        buffers.  With error feedback (:409-437) the EMA takes g + residual and
        the residual then takes the encoding loss delta - decode(new, alpha=0)
        (its EMA after the first step), in fp32 elementwise ops in the
        reference's order.  Returns m (fp32, shape of g)."""
        _require_gpu(g, "CoStateManager.update")
        _require_block_size(self.block_size)
        n = g.numel()
        if self._encoded is None or self._encoded["labels"].device != g.device:
            self.allocate(n, g.device)
        g32 = _f32_flat(g)
        if self._error_feedback and self._ef_residual is not None:
            m_hat = (_decode(self._encoded, self._alpha, g, n, True, False) if self._has_state
                     else torch.zeros(n, dtype=torch.float32, device=g.device))
            g_corrected = g32 + self._ef_residual.reshape(-1).float()
            m = beta1 * m_hat + (1.0 - beta1) * g_corrected
        else:
            m = _decode(self._encoded, self._alpha, g, n, self._has_state, True, beta1)
        alpha_new, delta = decompose(m, g32)
        ratios = compute_block_ratios(delta, m)
        tau0, tau1 = compute_thresholds(ratios, self._null_pct, self._amp_pct)
        labels = classify_blocks(ratios, tau0, tau1)
        enc = encode_blocks(delta, labels)
        if self._error_feedback:
            zero = torch.zeros(1, dtype=torch.float32, device=g.device)
            ef_error = delta.reshape(-1) - _decode(enc, zero, g, n, True, False)
            if self._ef_residual is None:
                self._ef_residual = ef_error.reshape(g.shape)
            else:
                self._ef_residual = (beta1 * self._ef_residual.reshape(-1).float()
                                     + (1.0 - beta1) * ef_error).reshape(g.shape)
        for k in ("labels", "sign_packed", "block_norms", "scales"):
            self._encoded[k].copy_(enc[k])
        if isinstance(self._alpha, torch.Tensor):
            self._alpha.copy_(alpha_new)
        else:
            self._alpha = alpha_new.clone()
        self._original_numel = n
        self._has_state = True
        return m.reshape(g.shape)
