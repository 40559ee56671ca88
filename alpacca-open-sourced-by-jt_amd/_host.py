"""Host-array adapters for the NumPy-facing drop-ins.

The reference's ``kernels``/``qwen35_kernels``/``cuda`` entry points take and
return host NumPy arrays.  Their drop-ins here accept either NumPy arrays
(uploaded to the current HIP device, result downloaded: the PCIe-inclusive
form) or torch device tensors (used in place, result stays on the device).
"""

from __future__ import annotations

import numpy as np


def torch_mod():
    import torch
    return torch


def device():
    torch = torch_mod()
    if not torch.cuda.is_available():
        from ._lib import AlpxUnavailable
        raise AlpxUnavailable("no HIP device is visible")
    return torch.device("cuda", torch.cuda.current_device())


def is_host(x) -> bool:
    return not (hasattr(x, "device") and hasattr(x, "data_ptr"))


def to_device(x, dtype=None):
    """NumPy -> contiguous device tensor (float32 unless it is fp16);
    device tensors pass through (made contiguous)."""
    torch = torch_mod()
    if is_host(x):
        arr = np.asarray(x)
        if arr.dtype not in (np.float16, np.float32):
            arr = arr.astype(np.float32)
        t = torch.from_numpy(np.ascontiguousarray(arr)).to(device())
    else:
        t = x.contiguous()
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t


def to_host(t):
    return t.float().cpu().numpy()
