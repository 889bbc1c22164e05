"""Loading checkpoints written by the reference package (davidkny22/turboadam).

A reference optimizer state dict pickles its per-parameter
`turboadam.costate.CoStateManager` objects (reference optimizer.py:242-248,
costate.py:357-365).  load_reference_checkpoint reads such a file with
torch's weights-only unpickler -- nothing in the file is executed -- and maps
that class name to this package's CoStateManager; TurboAdam.load_state_dict
then adopts the managers, restores the packed dtypes and drops `rand_buf`.
"""

import torch

from .costate import CoStateManager

REFERENCE_MANAGER = "turboadam.costate.CoStateManager"


def load_reference_checkpoint(f, map_location=None):
    """torch.load(f, weights_only=True) with the reference's CoStateManager
    allowed and loaded as turboadam_amd.costate.CoStateManager."""
    with torch.serialization.safe_globals([(CoStateManager, REFERENCE_MANAGER)]):
        return torch.load(f, map_location=map_location, weights_only=True)
