"""1Q second-moment state: initial state, compression and decode.

State dict layout (reference src/turboadam/oneq.py:41-48):
    {"indices": u8[nb*128], "scales": f16[nb, 2] (log_min, log_max),
     "n_bits": int, "original_shape": torch.Size, "original_length": int,
     "block_size": int}
"""

import torch

from . import _lib
from .quantize import DEFAULT_SEED, _dequantize_operands, quantize_logscale_nbits
from .utils import BLOCK_SIZE, num_blocks

# TurboAdam starts v from full(1e-30) quantised deterministically
# (reference optimizer.py:273-280 -> oneq.py:13-48 -> quantize.py:177-178):
# every element equals the block minimum, so every index is 0 and both block
# scales are f16(log(f32(1e-30))), computed here exactly as the reference does.
V_INIT_VALUE = 1e-30
V_INIT_SCALE = float(torch.tensor(V_INIT_VALUE, dtype=torch.float32).clamp(min=1e-38).log().to(torch.float16))


def init_v_state(param: torch.Tensor, n_bits: int, block_size: int = BLOCK_SIZE) -> dict:
    """First-step compressed v of `param` (the closed form of compress_v_logscale(full(1e-30)))."""
    n = param.numel()
    nb = num_blocks(n, block_size)
    dev = param.device
    return {
        "indices": torch.zeros(nb * block_size, dtype=torch.uint8, device=dev),
        "scales": torch.full((nb, 2), V_INIT_SCALE, dtype=torch.float16, device=dev),
        "n_bits": n_bits,
        "original_shape": param.shape,
        "original_length": n,
        "block_size": block_size,
    }


def compress_v_logscale(v: torch.Tensor, n_bits: int = 3, block_size: int = BLOCK_SIZE,
                        stochastic_round: bool = False, *, tensor_id: int = 0, step: int = 1,
                        seed: int = DEFAULT_SEED) -> dict:
    """Compress v into the 1Q state dict (reference oneq.py:13-48).

    The last block is filled up to block_size elements with the fp32 value
    max(min(v), 1e-38): padding can then neither lower the block's minimum
    nor (a log of zero) make it infinite.  That value is formed on the device
    (the reference reads min(v) back to the host first); the blocks then go
    through quantize_logscale_nbits."""
    flat = v.reshape(-1).to(torch.float32)
    count = flat.numel()
    blocks = torch.empty(num_blocks(count, block_size) * block_size, dtype=torch.float32, device=flat.device)
    blocks[:count] = flat
    if blocks.numel() > count:
        blocks[count:] = flat.min().clamp(min=1e-38)  # NaN stays NaN, as Python's max(nan, 1e-38)
    indices, scales, _ = quantize_logscale_nbits(blocks, n_bits=n_bits, block_size=block_size,
                                                 stochastic_round=stochastic_round, tensor_id=tensor_id,
                                                 step=step, seed=seed)
    return dict(indices=indices, scales=scales, n_bits=n_bits, original_shape=v.shape, original_length=count,
                block_size=block_size)


def decompress_v(compressed: dict) -> torch.Tensor:
    """Reconstruct fp32 v (reference oneq.py:51-67) with the gfx950 decode kernel."""
    idx = compressed["indices"]
    scales = compressed["scales"]
    if not idx.is_cuda:
        raise RuntimeError("turboadam_amd.decompress_v: state must be on an MI355X (HIP) device")
    if compressed["block_size"] != BLOCK_SIZE:
        raise NotImplementedError("turboadam_amd supports block_size=128 only")
    lib = _lib.load()
    idx, scales, n = _dequantize_operands(idx, scales, BLOCK_SIZE, compressed["original_length"])
    out = torch.empty(n, dtype=torch.float32, device=idx.device)
    with torch.cuda.device(idx.device):
        rc = lib.tam_v_dequantize(idx.data_ptr(), scales.data_ptr(), n, compressed["n_bits"], out.data_ptr(),
                                  _lib.stream_of(idx.device))
    _lib.check(rc, "tam_v_dequantize")
    return out.reshape(compressed["original_shape"])
