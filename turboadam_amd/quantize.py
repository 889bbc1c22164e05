"""1Q log-scale codec for the second moment (reference src/turboadam/quantize.py).

Per 128-element block: fp16 (log_min, log_max) and one uint8 index per
element; value = exp(log_min + ((idx + 0.5) / 2^bits) * (log_max - log_min)).
TurboAdam.step runs fused_v_update inside its multi-tensor pass; the
reference's public functions are also available one tensor at a time on the
gfx950 kernels, with the step's arithmetic (correctly rounded log and exp).

Stochastic rounding draws come from Philox4x32-10 keyed by (seed, tensor_id,
step) exactly as in the step, so the extra keyword arguments tensor_id, step
and seed replace the reference's torch.rand_like.
"""

import torch

from . import _lib
from .utils import BLOCK_SIZE, num_blocks

DEFAULT_SEED = 0x7A3D_5EED_0BAD_C0DE
_BITS = (2, 3, 4, 6, 8)


def _check(n_bits: int, block_size: int, t: torch.Tensor, what: str) -> None:
    if n_bits not in _BITS:
        raise ValueError(f"v_bits must be one of {_BITS}, got {n_bits}")
    if block_size != BLOCK_SIZE:
        raise NotImplementedError("turboadam_amd supports block_size=128 only")
    if not t.is_cuda:
        raise RuntimeError(f"turboadam_amd.{what}: tensors must be on an MI355X (HIP) device, got {t.device}")


def quantize_logscale_nbits(v_flat: torch.Tensor, n_bits: int = 3, block_size: int = BLOCK_SIZE,
                            stochastic_round: bool = False, *, tensor_id: int = 0, step: int = 1,
                            seed: int = DEFAULT_SEED):
    """Quantize a 1-D positive tensor whose length is a multiple of 128
    (reference quantize.py:126-180).  Returns (indices u8[n], scales f16[nb, 2], n_bits)."""
    _check(n_bits, block_size, v_flat, "quantize_logscale_nbits")
    assert v_flat.ndim == 1
    assert v_flat.shape[0] % block_size == 0
    lib = _lib.load()
    v = v_flat.float().contiguous()
    n = v.numel()
    dev = v.device
    idx = torch.empty(n, dtype=torch.uint8, device=dev)
    scales = torch.empty((n // block_size, 2), dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        _lib.check(lib.tam_v_quantize(v.data_ptr(), n, n_bits, int(bool(stochastic_round)), tensor_id, step, seed,
                                      idx.data_ptr(), scales.data_ptr(), _lib.stream_of(dev)), "tam_v_quantize")
    return idx, scales, n_bits


def _dequantize_operands(indices: torch.Tensor, scales: torch.Tensor, block_size: int, original_numel: int):
    """Contiguous u8 indices, f16 scales and the element count of a decode.

    As in the reference (quantize.py:202-214): the indices form (nb, 128) with
    nb = scales.shape[0], and the result is the first original_numel values
    (all nb*128 when 0; a larger count yields only the nb*128 that exist)."""
    nb = scales.shape[0] if scales.dim() > 0 else 0
    if scales.numel() != 2 * nb or indices.numel() != nb * block_size:
        raise RuntimeError(f"dequantize_logscale_nbits: {indices.numel()} indices and scales of shape "
                           f"{tuple(scales.shape)} do not form (num_blocks, {block_size}) blocks")
    n = original_numel or nb * block_size
    n = min(int(n), nb * block_size)
    return indices.to(torch.uint8).contiguous(), scales.to(torch.float16).contiguous(), n


def dequantize_logscale_nbits(indices: torch.Tensor, scales: torch.Tensor, n_bits: int = 3,
                              block_size: int = BLOCK_SIZE, original_numel: int = 0) -> torch.Tensor:
    """Values of a 1Q representation (reference quantize.py:183-214); fp32[original_numel]."""
    _check(n_bits, block_size, indices, "dequantize_logscale_nbits")
    lib = _lib.load()
    idx, sc, n = _dequantize_operands(indices, scales, block_size, original_numel)
    out = torch.empty(n, dtype=torch.float32, device=idx.device)
    with torch.cuda.device(idx.device):
        _lib.check(lib.tam_v_dequantize(idx.data_ptr(), sc.data_ptr(), n, n_bits, out.data_ptr(),
                                        _lib.stream_of(idx.device)), "tam_v_dequantize")
    return out


def fused_v_update(indices: torch.Tensor, scales: torch.Tensor, grad: torch.Tensor, beta2: float, n_bits: int,
                   block_size: int = BLOCK_SIZE, original_numel: int = None, *, tensor_id: int = 0, step: int = 1,
                   seed: int = DEFAULT_SEED):
    """Decode, v = beta2*v + (1-beta2)*g^2, re-quantize with stochastic rounding
    (reference quantize.py:222-299).  Returns (new_indices u8[nb*128],
    new_scales f16[nb, 2], v fp32[original_numel])."""
    _check(n_bits, block_size, grad, "fused_v_update")
    lib = _lib.load()
    g = grad.reshape(-1)
    if g.dtype not in _lib.DTYPES:
        g = g.float()
    g = g.contiguous()
    n = g.numel() if original_numel is None else original_numel
    nb = num_blocks(n)
    dev = g.device
    idx_in = indices.to(torch.uint8).contiguous()
    sc_in = scales.to(torch.float16).contiguous()
    if idx_in.numel() != nb * block_size or sc_in.numel() != 2 * nb:
        raise ValueError("fused_v_update: state does not match the gradient's block count")
    new_idx = torch.empty(nb * block_size, dtype=torch.uint8, device=dev)
    new_sc = torch.empty((nb, 2), dtype=torch.float16, device=dev)
    v = torch.empty(n, dtype=torch.float32, device=dev)
    b2 = float(torch.tensor(beta2, dtype=torch.float32))
    ob2 = float(torch.tensor(1.0 - beta2, dtype=torch.float32))
    with torch.cuda.device(dev):
        _lib.check(lib.tam_fused_v_update(idx_in.data_ptr(), sc_in.data_ptr(), g.data_ptr(), _lib.DTYPES[g.dtype], n,
                                          n_bits, b2, ob2, tensor_id, step, seed, new_idx.data_ptr(),
                                          new_sc.data_ptr(), v.data_ptr(), _lib.stream_of(dev)),
                   "tam_fused_v_update")
    return new_idx, new_sc, v
