"""Small shared helpers (reference: src/miniserve/utils.py:11-20)."""

from __future__ import annotations

from typing import Any

import numpy as np
import torch
from torch import Tensor


def to_device(data: Any, device: torch.device, dtype: torch.dtype = torch.long) -> Tensor:
    """Python data -> device tensor without stalling the host: staged through pinned memory and
    copied with non_blocking=True, so no hidden synchronization (utils.py:11-20)."""
    if device.type != "cuda":
        return torch.tensor(data, dtype=dtype, device=device)
    return torch.tensor(data, dtype=dtype, pin_memory=True).to(device, non_blocking=True)


def upload_int32(arr: np.ndarray, device: torch.device) -> Tensor:
    """A host int32 array -> device tensor through pinned memory, non-blocking (as to_device)."""
    t = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.int32))
    if device.type != "cuda":
        return t.to(device)
    return t.pin_memory().to(device, non_blocking=True)
