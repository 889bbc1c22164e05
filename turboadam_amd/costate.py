"""CoState first-moment state (reference src/turboadam/costate.py:332-464).

m = alpha*g + delta is stored as one fp32 alpha per tensor plus, per
128-element block, a label (0 null, 1 phase, 2 amplitude), the residual L2
norm (fp32), an fp16 amplitude scale and one sign bit per element (MSB first).
The update itself runs fused inside TurboAdam.step on the GPU; this class
keeps the reference's per-tensor state object and attribute names so saved
state and inspection code see the same layout.
"""

import torch

from .utils import BLOCK_SIZE, num_blocks


class CoStateManager:
    """Per-tensor CoState state (same attributes as the reference, costate.py:350-365)."""

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
        """Sorted positions of the two thresholds (costate.py:115-117, Python double arithmetic)."""
        lo = max(0, int(self._null_pct * nb) - 1)
        hi = min(nb - 1, int(self._amp_pct * nb))
        return lo, hi

    def update(self, g: torch.Tensor, beta1: float) -> torch.Tensor:
        raise NotImplementedError(
            "turboadam_amd runs the CoState update fused inside TurboAdam.step (one multi-tensor launch); "
            "a standalone per-tensor update is not provided"
        )
