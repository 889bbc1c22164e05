"""Block helpers the 1Q initialisation uses (reference src/turboadam/utils.py:27-53)."""

import torch

BLOCK_SIZE = 128


def pad_to_blocks(tensor: torch.Tensor, block_size: int = BLOCK_SIZE, pad_value: float = 0.0):
    """Pad a flat 1-D tensor to the next multiple of block_size.

    Same contract as the reference (utils.py:27-53): returns
    (padded, original_length); a tensor whose length is already a multiple of
    block_size is returned unchanged (no copy).
    """
    original_length = tensor.shape[0]
    remainder = original_length % block_size
    if remainder == 0:
        return tensor, original_length
    fill = tensor.new_full((block_size - remainder,), pad_value)
    return torch.cat([tensor, fill]), original_length


def num_blocks(n: int, block_size: int = BLOCK_SIZE) -> int:
    return (n + block_size - 1) // block_size
