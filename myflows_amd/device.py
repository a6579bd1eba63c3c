"""Device selection for the framework's arrays (torch tensors).

Mirrors the reference's global CPU/CUDA switch (``core/device.py:146-170``): parameters and inputs
are created on the active device. The ``hip_native`` operators run only on the GPU; handing them CPU
tensors raises the same ``ValueError`` the reference raises for a native backend on the CPU device.
"""

from __future__ import annotations

import torch

_DEVICE = "cuda" if torch.cuda.is_available() else "cpu"


def cuda_available() -> bool:
    return torch.cuda.is_available()


def get_device() -> str:
    return _DEVICE


def set_device(device: str) -> str:
    global _DEVICE
    name = str(device).strip().lower()
    if name == "cpu":
        _DEVICE = "cpu"
    elif name in ("cuda", "gpu", "hip", "cuda:0"):
        if not torch.cuda.is_available():
            raise RuntimeError("a GPU was requested but none is visible")
        _DEVICE = "cuda"
    else:
        raise ValueError(f"unsupported device {device!r}; use 'cpu' or 'cuda'")
    return _DEVICE


def torch_device():
    return torch.device("cuda", torch.cuda.current_device()) if _DEVICE == "cuda" else torch.device("cpu")


def asarray(value, dtype=torch.float32):
    """A tensor on the active device (numpy arrays and Python values are copied there)."""
    if isinstance(value, torch.Tensor):
        return value.to(device=torch_device(), dtype=dtype)
    return torch.as_tensor(value, dtype=dtype, device=torch_device())
